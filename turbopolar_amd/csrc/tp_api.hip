// tp_api.hip -- error reporting, version and layout rules of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "tp_common.h"

namespace tp {

static thread_local char g_error[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_error[0] = 0; }

// Validates the layout against the encoder's supported bit widths
// (rfsn_v11/quant/polar/encoder.py:56-83) and the config's split_dim rule
// (rfsn_v11/candidates/turbo_polar_config.py:50-51).
bool check_layout(const tp_page_layout* layout, int* l1_row, int* deep_row) {
  if (!layout) {
    set_error("layout is NULL");
    return false;
  }
  if (layout->l1_bits != 4 && layout->l1_bits != 8) {
    set_error("unsupported k_angle_bits_level1: %d", layout->l1_bits);
    return false;
  }
  if (layout->deep_bits != 2 && layout->deep_bits != 4 && layout->deep_bits != 8) {
    set_error("unsupported k_angle_bits_deep: %d", layout->deep_bits);
    return false;
  }
  if (layout->split_dim < 0 || layout->split_dim > kHeadDim || (layout->split_dim & 1)) {
    set_error("split_dim must be even and within [0, head_dim]");
    return false;
  }
  if (layout->int8_radii != 0 && layout->int8_radii != 1) {
    set_error("int8_radii must be 0 or 1");
    return false;
  }
  const int split_half = layout->split_dim / 2;
  if (l1_row) *l1_row = packed_row_bytes(split_half, layout->l1_bits);
  if (deep_row) *deep_row = packed_row_bytes(kPairs - split_half, layout->deep_bits);
  return true;
}

int32_t launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: %s", what, hipGetErrorString(e));
    return TP_ERR_HIP;
  }
  return TP_OK;
}

}  // namespace tp

extern "C" {

const char* tp_last_error(void) { return tp::g_error; }

int32_t tp_version(void) { return 100; }

int32_t tp_layout_row_bytes(const tp_page_layout* layout, int32_t* l1_row_bytes,
                            int32_t* deep_row_bytes) {
  tp::clear_error();
  int l1 = 0, deep = 0;
  if (!tp::check_layout(layout, &l1, &deep)) return TP_ERR_UNSUPPORTED;
  if (l1_row_bytes) *l1_row_bytes = l1;
  if (deep_row_bytes) *deep_row_bytes = deep;
  return TP_OK;
}

}  // extern "C"
