/*
 * turbopolar.h -- C ABI of the MI355X (gfx950) TurboPolar compressed-KV
 * decode-attention library (libturbopolar_hip.so).
 *
 * The library replaces the reference's kernel bridge
 * (rfsn_v11/kernels/turbo_polar/metal.py, class MetalKernelBridge) and the
 * MLX-op codecs it calls.  Every entry point takes plain device pointers and
 * sizes, is stream-ordered and asynchronous (no host synchronisation), never
 * allocates device memory, and returns a status code (TP_OK on success);
 * tp_last_error() returns the message of the last failure on the calling
 * thread.
 *
 * Page layout (one page = 64 tokens of one (batch, kv-head); "bh" below is
 * batch * num_kv_heads + kv_head).  It is the structure-of-arrays layout of
 * PolarKBlockStorage / QuantVBlockStorage (rfsn_v11/generation/storage.py:17-169),
 * with `capacity` page slots per bh:
 *   radii        [bh][capacity][64][64]  fp16, or int8 log-radius codes
 *   radii_scales [bh][capacity]          fp16, int8 layout only (else NULL)
 *   angle_l1     [bh][capacity][64][l1_row_bytes]    uint8, packed
 *   angle_deep   [bh][capacity][64][deep_row_bytes]  uint8, packed
 *   v_codes      [bh][capacity][64][128] int8
 *   v_scales     [bh][capacity][64][4]   fp16 (one per group of 32 dims)
 */
#ifndef TURBOPOLAR_H_
#define TURBOPOLAR_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TP_PAGE_TOKENS 64
#define TP_HEAD_DIM 128
/* Static split-K scratch per GPU of tp_decode_attention_noalloc. */
#define TP_NOALLOC_SCRATCH_BYTES ((size_t)8 << 20)

/* Status codes.  The Python shim maps TP_ERR_INVALID to ValueError and the
 * others to RuntimeError, mirroring the reference's exception contract. */
enum {
  TP_OK = 0,
  TP_ERR_INVALID = 1,     /* bad argument (shape, pointer, size) */
  TP_ERR_UNSUPPORTED = 2, /* layout the kernels do not implement */
  TP_ERR_HIP = 3,         /* HIP launch/runtime error */
  TP_ERR_WORKSPACE = 4,   /* workspace missing or too small */
  TP_ERR_NONFINITE = 5    /* tp_append_stage: the input holds NaN or inf */
};

/* Compression layout of the key codes; the fields of TurboPolarConfig that
 * fix the page format (rfsn_v11/candidates/turbo_polar_config.py:11-21) and the
 * encoder's metadata (rfsn_v11/quant/polar/encoder.py:85-97). */
typedef struct tp_page_layout {
  int32_t int8_radii; /* 0: fp16 radii; 1: int8 log radii + fp16 page scale */
  int32_t l1_bits;    /* 4 or 8: angle bits of pairs [0, split_dim/2) */
  int32_t deep_bits;  /* 2, 4 or 8: angle bits of pairs [split_dim/2, 64) */
  int32_t split_dim;  /* even, 0..128 */
} tp_page_layout;

/* Device pointers of one page store (see the layout above).  The attention
 * entry points read radii, angle_deep and v_codes in 16-byte, angle_l1 in
 * 8-byte and v_scales in 4-byte units, and reject buffers aligned less (any
 * device allocation, and any page slot of one, is aligned enough). */
typedef struct tp_pages {
  void* radii;
  void* radii_scales;
  uint8_t* angle_l1;
  uint8_t* angle_deep;
  int8_t* v_codes;
  void* v_scales;
  int64_t capacity; /* page slots per bh */
} tp_pages;

/* QJL residual sketches of the pages (no counterpart struct in the reference:
 * it passes QJLPayload.packed_signs / norms and q_proj_signs as separate
 * arrays, metal.py:532-571).  signs: uint8 [bh][capacity][64][proj_dim / 8],
 * one sketch per token, page p of row bh in slot bh * capacity + p as in the
 * page store; norms: fp16 [bh][capacity][64] residual norms; q_signs: uint8
 * [batch][hq][proj_dim / 8] sketches of the queries.  proj_dim: a multiple of
 * 8 from 8 to 256 (turbo_polar_config.py:34-37 takes any positive multiple of
 * 8).  Alignment: proj_dim == 64 (the kernels' 64-bit path) signs 16-byte,
 * norms and q_signs 8-byte; any other width signs 4-byte, norms 2-byte. */
typedef struct tp_qjl {
  const void* signs;
  const void* norms;
  const void* q_signs;
  int32_t proj_dim;
  int64_t capacity; /* sketch page slots per bh (>= n_pages) */
} tp_qjl;

/* Last error message of the calling thread ("" if none). */
const char* tp_last_error(void);

/* Library ABI version (major * 100 + minor). */
int32_t tp_version(void);

/* Packed bytes per token of the l1 and deep angle-code rows.  Restates the
 * packed shapes of PolarQuantEncoder._pack_4bit/_pack_2bit
 * (rfsn_v11/quant/polar/encoder.py:56-83,101-130). */
int32_t tp_layout_row_bytes(const tp_page_layout* layout, int32_t* l1_row_bytes,
                            int32_t* deep_row_bytes);

/*
 * Encode pages: polar keys + grouped int8 values.
 * Replaces PolarQuantEncoder.encode_block (rfsn_v11/quant/polar/encoder.py:24-98)
 * and GroupedVQuantizer.quantize_block (rfsn_v11/quant/v_quant/encoder.py:16-30)
 * as called by TurboPolarKVCacheRuntime._flush_block / _maybe_encode_partial
 * (rfsn_v11/generation/turbo_polar_cache.py:128-161,276-319).
 *
 * k, v: [bh][in_tokens][128], fp16 (in_dtype 0) or fp32 (in_dtype 1); either may
 * be NULL to encode only the other.  Tokens [token_begin, token_begin+n_tokens)
 * are encoded into page slots [page_begin, page_begin + ceil(n_tokens/64)) of
 * `pages`; a last partial page is zero-padded (as _maybe_encode_partial does).
 * Codes and scales are bit-exact with the reference encoder's fp16 semantics.
 */
int32_t tp_encode_pages(const void* k, const void* v, int32_t in_dtype, int64_t bh,
                        int64_t in_tokens, int64_t token_begin, int64_t n_tokens,
                        const tp_page_layout* layout, const tp_pages* pages,
                        int64_t page_begin, void* stream);

/*
 * Fused dequant . QK scores over all n_pages*64 page slots (no masking).
 * Replaces MetalKernelBridge.execute_fused_qk (metal.py:494-530) and its kernel
 * tqpolar_fused_dequant_qk (tqpolar_fused_qk.metal:4-100).
 * q: fp16 [batch][hq][128]; scores: fp16 [batch][hq][n_pages*64], 16-byte
 * aligned.
 * scale is applied in fp32 (the shim passes fp16(attention_scale), as
 * metal.py:518 does).
 */
int32_t tp_fused_qk(const void* q, int64_t batch, int32_t hq, int32_t hkv,
                    const tp_page_layout* layout, const tp_pages* pages, int32_t n_pages,
                    float scale, void* scores, void* stream);

/*
 * Split-K decode attention over compressed pages plus an optional dense tail.
 * Replaces MetalKernelBridge.execute_online_attention_quant_v (metal.py:651-715)
 * and execute_online_attention_quant_v_dense_tail (metal.py:717-792), kernels
 * tqpolar_online_attention_quant_v[_dense_tail]
 * (tqpolar_online_attention.metal:197-390,393-629).
 *
 * q: fp16 [batch][hq][128]; out: fp16 [batch][hq][128].
 * tail_k, tail_v: fp16 [batch][hkv][tail_stride][128] holding tail_len (0..63)
 *   dense tokens that follow the pages (NULL when tail_len == 0).
 * Tokens with global index >= actual_seq_len are masked (actual_seq_len >= 1;
 *   a value past the stored tokens attends every stored token, as the
 *   reference's mask does).
 * pages_per_split: pages per workgroup (0 = library default); the grid is
 *   (hkv, batch x ceil(hq / hkv / 16), ceil(n_pages / pages_per_split))
 *   workgroups, and its second and third sizes must not exceed 65535.
 * workspace: device memory of at least tp_decode_workspace_bytes(...) bytes.
 *   Its counter area (the first tp_decode_counter_bytes(batch, hq, hkv) bytes)
 *   must be zero before the first call; every call leaves it zero again.  One
 *   workspace must not be used by two calls that can run concurrently.
 */
int32_t tp_decode_attention(const void* q, int64_t batch, int32_t hq, int32_t hkv,
                            const tp_page_layout* layout, const tp_pages* pages,
                            int32_t n_pages, const void* tail_k, const void* tail_v,
                            int32_t tail_len, int64_t tail_stride, int64_t actual_seq_len,
                            float scale, int32_t pages_per_split, void* workspace,
                            size_t workspace_bytes, void* out, void* stream);

/*
 * tp_decode_attention without a workspace argument: allocates nothing (no
 * hipMalloc, hipFree or allocating library call).  No counterpart in the
 * reference; it is for callers that cannot allocate device memory: code under
 * HIP graph capture, tight serving loops, harnesses that forbid allocation.
 * The split-K records and ticket counters live in a static device scratch
 * array of TP_NOALLOC_SCRATCH_BYTES (8 MiB) per GPU, held until the
 * process ends.  A call whose tp_decode_workspace_bytes(...) exceeds it
 * returns TP_ERR_WORKSPACE (raise pages_per_split, or use
 * tp_decode_attention).  All calls on one GPU share that GPU's scratch, so
 * calls that can run concurrently on one GPU (other streams, other threads)
 * race; calls on one stream are ordered and safe.  The first call on a GPU
 * looks up the scratch address and clears its counter area with a kernel on
 * `stream`.  Other arguments, results and errors as tp_decode_attention.
 */
int32_t tp_decode_attention_noalloc(const void* q, int64_t batch, int32_t hq, int32_t hkv,
                                    const tp_page_layout* layout, const tp_pages* pages,
                                    int32_t n_pages, const void* tail_k, const void* tail_v,
                                    int32_t tail_len, int64_t tail_stride, int64_t actual_seq_len,
                                    float scale, int32_t pages_per_split, void* out, void* stream);

/* Workspace size for tp_decode_attention (same arguments). */
size_t tp_decode_workspace_bytes(int64_t batch, int32_t hq, int32_t hkv, int32_t n_pages,
                                 int32_t tail_len, int32_t pages_per_split);

/* Size of the zero-initialised counter area at the start of the workspace:
 * 64 KiB for up to 16384 units (batch x hkv x ceil(hq / hkv / 16)), 4 bytes
 * per unit beyond.  Up to that size it is the same for every shape, so one
 * workspace, zeroed once, serves calls of any shape. */
size_t tp_decode_counter_bytes(int64_t batch, int32_t hq, int32_t hkv);

/* Host-side bounds check of the decode kernels (no GPU work, no counterpart in
 * the reference): for one launch of tp_decode_attention (kernel 0; with
 * qjl != 0 tp_decode_attention_qjl, with dense_v != 0
 * tp_decode_attention_dense_v) or tp_fused_qk (kernel 1) of this shape,
 * enumerates every workgroup's, wave's and lane's global loads and stores --
 * page fields, q, the dense tail, QJL sketches, dense V, split-K records,
 * tickets and the output -- from the kernels' own address functions, and
 * returns how many fall outside their buffers (msg: the first of them).
 * Buffers take the smallest sizes the ABI admits: page fields of `capacity`
 * slots per bh, the dense tail ending right after the last row's tail_len
 * tokens, the workspace of tp_decode_workspace_bytes.  mutate is a test hook
 * that plants a known fault in the enumeration only: 1 moves every lane's
 * second V-scale dword 512 bytes on (one page's scales), 2 points a wave
 * without a page at the next split's first page instead of its own split's. */
typedef struct tp_bounds_case {
  int64_t batch;
  int32_t hq;
  int32_t hkv;
  tp_page_layout layout;
  int32_t n_pages;
  int64_t capacity;
  int32_t tail_len;
  int64_t tail_stride;
  int64_t seq_len;
  int32_t pages_per_split;
  int32_t qjl;
  int64_t qjl_capacity;
  int32_t dense_v;
  int64_t v_capacity;
  int32_t kernel;
  int32_t mutate;
  int32_t qjl_bits; /* QJL sketch bits (0 reads as 64) */
} tp_bounds_case;
unsigned long long tp_selftest_decode_bounds(const tp_bounds_case* c, char* msg, int32_t msg_len);

/* Pages per workgroup that tp_decode_attention uses when given 0. */
int32_t tp_default_pages_per_split(int64_t batch, int32_t hq, int32_t hkv, int32_t n_pages);

/*
 * Decode pages back to dense fp16 K and V (decompress-on-read).
 * Replaces PolarQuantDecoder.decode_block (rfsn_v11/quant/polar/decoder.py:7-67)
 * and GroupedVQuantizer.dequantize_block (rfsn_v11/quant/v_quant/encoder.py:32-38).
 * k_out, v_out: fp16 [bh][n_pages*64][128] (either may be NULL).
 */
int32_t tp_decode_pages(const tp_page_layout* layout, const tp_pages* pages, int64_t bh,
                        int64_t page_begin, int32_t n_pages, void* k_out, void* v_out,
                        void* stream);

/* tp_decode_pages into rows of a larger output: k_out, v_out are fp16
 * [bh][out_tokens][128] and page page_begin + p of row r lands at tokens
 * [out_offset + 64 p, out_offset + 64 p + 64) of row r (out_offset + 64 n_pages
 * <= out_tokens).  The decompress-on-read path decodes the stored pages and
 * the zero-padded tail page (turbo_polar_cache.py:200-274) side by side into
 * one buffer with it.  Same replaced functions as tp_decode_pages. */
int32_t tp_decode_pages_into(const tp_page_layout* layout, const tp_pages* pages, int64_t bh,
                             int64_t page_begin, int32_t n_pages, void* k_out, void* v_out,
                             int64_t out_tokens, int64_t out_offset, void* stream);

/* Selected pages in one launch: output page j of every (batch, head) row is
 * stored page page_index[j] (page_index: device int32 array of n_index
 * entries; entries outside [0, n_stored) are clamped into it, so the launch
 * never reads past the first n_stored pages -- callers check the indices
 * first).  k_out, v_out: fp16 [bh][n_index*64][128] (either may be NULL).
 * Replaces the per-page decode_block loop of
 * TurboPolarKVCacheRuntime.fetch_blocks (turbo_polar_cache.py:321-346). */
int32_t tp_decode_pages_gather(const tp_page_layout* layout, const tp_pages* pages, int64_t bh,
                               int32_t n_stored, const int32_t* page_index, int32_t n_index, void* k_out,
                               void* v_out, void* stream);

/* Append staging (replaces the per-input mx.isfinite(...).all() check of
 * TurboPolarKVCacheRuntime._validate_append_inputs, turbo_polar_cache.py:69,
 * and the dense-tail concatenation of append, :114-115).
 *
 * k, v: [bh][in_tokens][128] of in_dtype (0 fp16, 1 fp32), 16-byte aligned.
 * Copies tokens [copy_begin, copy_begin + n_copy) of every (b, h) row into
 * tail_k / tail_v ([bh][tail_tokens][128], same dtype) at token tail_pos.
 * With check != 0 it also scans every element of k and v; the kernel stores
 * `epoch` into *flag if any is NaN or inf, and this call then synchronises
 * `stream`, reads the flag and returns TP_ERR_NONFINITE, or TP_OK.  check == 1:
 * flag is caller-owned device memory, read back with a 4-byte copy.  check == 2:
 * flag is caller-owned pinned host memory from hipHostMalloc (device-visible)
 * and epoch must be even; the kernel writes epoch + 1 there on a non-finite
 * value with system-scope stores, and when the launch is a single workgroup
 * (up to 16 token rows of 128 fp16 or 8 of fp32) it also reports completion
 * itself (epoch or epoch + 1), so the call polls the flag instead of
 * synchronising the stream (bounded, then synchronising).  Pass a fresh epoch
 * per call so the flag never needs clearing.  check == 3 (deferred verdict, no
 * counterpart in the reference): as check == 2, but the call returns after the
 * launch and the kernel only ever writes epoch + 1 (on a non-finite value);
 * the caller reads the flag once the stream has passed the launch.  With
 * check == 0 or 3 the call is asynchronous like the others. */
int32_t tp_append_stage(const void* k, const void* v, int32_t in_dtype, int64_t bh, int64_t in_tokens,
                        int64_t copy_begin, int64_t n_copy, void* tail_k, void* tail_v, int64_t tail_tokens,
                        int64_t tail_pos, int32_t check, uint32_t* flag, uint32_t epoch, void* stream);

/* ---- QJL (rejected by TurboPolarConfig, turbo_polar_config.py:46-47, as in
 * the reference; these serve the bridge-level QJL calls the reference's own
 * tests make). ---- */

/* QJLResidualEncoder.compute_residual_sketch (rfsn_v11/quant/qjl/encoder.py:
 * 30-44) and the query sketch (q @ W >= 0, packed): e [rows][dim] of in_dtype
 * (0 fp16, 1 fp32), w fp32 [dim][proj_dim] -> packed uint8 [rows][proj_dim / 8]
 * (bit i of byte j: projection 8j + i >= 0) and, if norms is not NULL, fp16
 * [rows] = f16(sqrt(sum e^2)).  dim <= 256, proj_dim a multiple of 8 up to 256. */
int32_t tp_qjl_sketch(const void* e, int32_t in_dtype, int64_t rows, int32_t dim, const float* w, int32_t proj_dim,
                      uint8_t* packed, uint16_t* norms, void* stream);

/* qjl_dot_estimate (rfsn_v11/quant/qjl/score_estimate.py:6-54): out fp32
 * [batch][hq][tokens] = norms[kv][t] * |q[h]| * sin(pi/2 (P - 2 hamming) / P),
 * kv = h / (hq / hkv); q fp16 [batch][hq][dim], k_packed uint8
 * [batch][hkv][tokens][P / 8], norms fp16 [batch][hkv][tokens], q_packed uint8
 * [batch][hq][P / 8]. */
int32_t tp_qjl_dot_estimate(const void* q, int64_t batch, int32_t hq, int32_t hkv, int32_t dim, const void* k_packed,
                            const void* norms, int64_t tokens, const void* q_packed, int32_t proj_dim, float* out,
                            void* stream);

/* tp_fused_qk plus the QJL correction * scale (MetalKernelBridge.
 * execute_fused_qk_qjl, metal.py:532-571, kernel tqpolar_fused_dequant_qk_qjl,
 * tqpolar_fused_qk.metal:102-233). */
int32_t tp_fused_qk_qjl(const void* q, int64_t batch, int32_t hq, int32_t hkv, const tp_page_layout* layout,
                        const tp_pages* pages, int32_t n_pages, const tp_qjl* qjl, float scale, void* scores,
                        void* stream);

/* tp_decode_attention with the QJL correction added to the page tokens'
 * scores (execute_online_attention_quant_v[_dense_tail] with use_qjl=True,
 * metal.py:651-792, kernel branches tqpolar_online_attention.metal:256-345 and
 * 459-545; the dense tail gets no correction, metal.py:310-316).  Same
 * arguments as tp_decode_attention plus qjl. */
int32_t tp_decode_attention_qjl(const void* q, int64_t batch, int32_t hq, int32_t hkv,
                                const tp_page_layout* layout, const tp_pages* pages, int32_t n_pages,
                                const tp_qjl* qjl, const void* tail_k, const void* tail_v, int32_t tail_len,
                                int64_t tail_stride, int64_t actual_seq_len, float scale,
                                int32_t pages_per_split, void* workspace, size_t workspace_bytes,
                                void* out, void* stream);

/* Decode attention over compressed K pages and dense fp16 V
 * (MetalKernelBridge.execute_online_attention_dense_v, metal.py:586-649,
 * kernel tqpolar_online_attention_dense_v, tqpolar_online_attention.metal:10-196;
 * the reference's dense_v_debug storage).  pages: the K fields only (v_codes
 * and v_scales are not read); v_dense: fp16 [batch*hkv][v_capacity][64][128],
 * 16-byte aligned, v_capacity >= n_pages; qjl: NULL, or the sketches for
 * use_qjl=True.  No dense tail (the reference's method takes none); n_pages >=
 * 1.  Other arguments, workspace and errors as tp_decode_attention. */
int32_t tp_decode_attention_dense_v(const void* q, int64_t batch, int32_t hq, int32_t hkv,
                                    const tp_page_layout* layout, const tp_pages* pages, int32_t n_pages,
                                    const tp_qjl* qjl, const void* v_dense, int64_t v_capacity,
                                    int64_t actual_seq_len, float scale, int32_t pages_per_split, void* workspace,
                                    size_t workspace_bytes, void* out, void* stream);

/* GroupedVQuantizer.quantize_block (rfsn_v11/quant/v_quant/encoder.py:16-30)
 * for any group size dividing the row: v is [rows][dim] of in_dtype (0 fp16,
 * 1 fp32); codes int8 [rows][dim], scales fp16 [rows][dim / group_size].  The
 * page encoder covers groups of 32 over 128 dims; this covers the rest. */
int32_t tp_quantize_v_groups(const void* v, int32_t in_dtype, int64_t rows, int32_t dim, int32_t group_size,
                             int8_t* codes, uint16_t* scales, void* stream);

/* The int8 log radii of PolarQuantEncoder.encode_block with use_int8_radii
 * (rfsn_v11/quant/polar/encoder.py:34-42) over a block of any length, one
 * scale per row: radii fp16 [rows][n] (n = tokens x 64 pairs) -> codes int8
 * [rows][n], scales fp16 [rows].  The page encoder covers 64-token blocks. */
int32_t tp_log_radii_rows(const void* radii, int64_t rows, int64_t n, int8_t* codes, uint16_t* scales,
                          void* stream);

/* ---- Self-test hooks: no counterpart in the reference.  They evaluate the
 * encoder's scalar fp16 helpers so tests can check them exhaustively, and
 * the decode kernel's host-side index arithmetic. ---- */

/* Host only (no GPU needed): for every divisor d in [1, d_max], checks the
 * decode kernel's multiply-shift division (the constants tp_decode_attention
 * passes for its workgroup-index divisions) against n / d at the ends of the
 * 31-bit dividend range, around multiples of d spread over it, and for the
 * first 3d + 5 dividends.  Returns the number of mismatches; *checks (if not
 * NULL) receives the number of dividends checked. */
unsigned long long tp_selftest_fastdiv(uint32_t d_max, unsigned long long* checks);

/* For every 16-bit pattern b: sqrt_out[b] = fp16 sqrt of b, log_out[b] = fp16
 * log(max(b, fp16(1e-6))), codes_out[3*b + {0,1,2}] = angle code of the fp16
 * angle b for 2, 4 and 8 bits (fp16 input rules). */
int32_t tp_selftest_f16_tables(uint16_t* sqrt_out, uint16_t* log_out, uint8_t* codes_out,
                               void* stream);

/* Counts, over x bit patterns [x_begin, x_begin+x_count) and all 65536 y
 * patterns (finite values only), the pairs where the encoder's fast fp16
 * atan2 differs from the float64 reference path, or where the 4- or 8-bit
 * angle code of the specialised fp16 encoder differs from the code of the
 * float64 angle.  *mismatches is accumulated (atomic add), so zero it first. */
int32_t tp_selftest_atan2_exhaustive(unsigned long long* mismatches, int32_t x_begin,
                                     int32_t x_count, void* stream);

/* Counts, over positive fp16 scale patterns [s_begin, s_begin+s_count) and all
 * 65536 value patterns (finite values only), the quotients where the V
 * quantiser's reciprocal-product fp16 division differs from the correctly
 * rounded one.  *mismatches is accumulated (atomic add), so zero it first. */
int32_t tp_selftest_div_f16_exhaustive(unsigned long long* mismatches, int32_t s_begin,
                                       int32_t s_count, void* stream);

/* Counts, over positive finite fp16 scale patterns [s_begin, s_begin+s_count)
 * and all finite fp16 values, the int8 V codes where the fast encoder's path
 * (reciprocal-product quotient, biased byte conversion, exact redo near an
 * fp16 midpoint) differs from int8(clip(rint(fp16(v / s)), -128, 127)).
 * *mismatches is accumulated (atomic add), so zero it first. */
int32_t tp_selftest_vcode_exhaustive(unsigned long long* mismatches, int32_t s_begin,
                                     int32_t s_count, void* stream);

/* Counts, over positive finite fp16 scale patterns [s_begin, s_begin+s_count)
 * and all finite fp16 log radii lr with |lr / scale| < 127.1, the int8
 * log-radius codes where the fast encoder's path (reciprocal FMA with the
 * +128 bias, byte conversion, exact redo near a half-integer) differs from
 * int8(clip(rint(f32(lr / scale)), -128, 127)).  *mismatches is accumulated
 * (atomic add), so zero it first.  Test-only, as the other self-tests. */
int32_t tp_selftest_lcode_exhaustive(unsigned long long* mismatches, int32_t s_begin,
                                     int32_t s_count, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TURBOPOLAR_H_ */
