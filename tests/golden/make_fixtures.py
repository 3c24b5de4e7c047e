"""Writes the golden fixtures in this directory from the NumPy oracle.

Run from the repository root:  python tests/golden/make_fixtures.py

The reference's own tests hold no data files for this path (they draw inputs
from ``mx.random`` at run time and check tolerances only), so the fixtures are
built from this suite's seeded generators (tests/common.py) and the oracle's
restatement of encoder.py:24-130, v_quant/encoder.py:16-38, decoder.py:7-85
and metal.py:254-332.  They freeze the oracle's answers so that the GPU kernels
and any later oracle change are checked against the same bytes.

Files:
  inputs.npz         K/V pages (1 x 2 kv heads x 2 pages), a 63-token dense
                     tail, queries for GQA 1/4/8, the edge page in fp16/fp32
  layout_<name>.npz  for the default and fast layouts: encoded page buffers,
                     decoded K/V (fp16), attention outputs (fp64 rounded to
                     fp32) for tails 0/1/37/63, GQA 1/4/8, and one masked
                     suffix; edge-page codes for fp16 and fp32 inputs
  edge_<name>.npz    edge-page codes for the deep2 and l1_8bit layouts
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
sys.path.insert(0, str(HERE.parent.parent))

import oracle  # noqa: E402
from common import LAYOUTS, PAGE, edge_page, gen_kv, gen_q, oracle_pages  # noqa: E402

SCALE16 = oracle.fp16_scale(1.0 / np.sqrt(128.0))
HKV = 2
S = 2
TAILS = (0, 1, 37, 63)
GQA = (1, 4, 8)
MASKED_SEQ = 100  # two pages, no tail, tokens 100..127 masked
SEED = 1


def make_inputs():
    k, v = gen_kv(SEED, 1, HKV, S * PAGE + max(TAILS), "normal", np.float16)
    out = {
        "k": k[:, :, : S * PAGE], "v": v[:, :, : S * PAGE],
        "tail_k": k[:, :, S * PAGE:], "tail_v": v[:, :, S * PAGE:],
    }
    for g in GQA:
        out[f"q_g{g}"] = gen_q(SEED + g, 1, HKV * g)
    for dt in (np.float16, np.float32):
        ek, ev = edge_page(dt)
        out[f"edge_k_{np.dtype(dt).name}"] = ek
        out[f"edge_v_{np.dtype(dt).name}"] = ev
    return out


def encode_fields(k, v, layout, prefix=""):
    blk, (vc, vs) = oracle_pages(k, v, layout)
    out = {
        prefix + "radii": blk["radii"],
        prefix + "angle_codes_l1": blk["angle_codes_l1"],
        prefix + "angle_codes_deep": blk["angle_codes_deep"],
        prefix + "v_codes": vc,
        prefix + "v_scales": vs,
    }
    if layout[0]:
        out[prefix + "radii_scales"] = blk["radii_scales"]
    return out, blk, (vc, vs)


def make_layout(name, inp):
    layout = LAYOUTS[name]
    out, blk, qv = encode_fields(inp["k"], inp["v"], layout)
    out["layout"] = np.array([int(layout[0]), layout[1], layout[2], layout[3]], np.int32)
    kd = oracle.decode_block(blk["radii"], blk["radii_scales"], blk["angle_codes_l1"], blk["angle_codes_deep"],
                             blk["metadata"])
    out["k_decoded"] = kd
    out["v_decoded"] = oracle.dequantize_block(*qv).reshape(kd.shape)
    for g in GQA:
        q = inp[f"q_g{g}"]
        for t in TAILS:
            res = oracle.cpu_online_attention_dense_tail(
                q, blk, qv, inp["tail_k"][:, :, :t], inp["tail_v"][:, :, :t], SCALE16, S * PAGE + t)
            out[f"out_g{g}_t{t}"] = res.astype(np.float32)
    out["out_g4_masked"] = oracle.cpu_online_attention(inp["q_g4"], blk, qv, SCALE16, MASKED_SEQ).astype(np.float32)
    return out


def make_edge(name, inp):
    out = {}
    for dt in ("float16", "float32"):
        fields, _, _ = encode_fields(inp[f"edge_k_{dt}"], inp[f"edge_v_{dt}"], LAYOUTS[name], prefix=f"{dt}__")
        out.update(fields)
    return out


def build_all():
    inp = make_inputs()
    files = {"inputs.npz": inp}
    for name in ("default", "fast"):
        files[f"layout_{name}.npz"] = {**make_layout(name, inp), **make_edge(name, inp)}
    for name in ("deep2", "l1_8bit"):
        files[f"edge_{name}.npz"] = make_edge(name, inp)
    return files


def main():
    for fname, arrays in build_all().items():
        np.savez_compressed(HERE / fname, **arrays)
        print(f"{fname}: {len(arrays)} arrays, {(HERE / fname).stat().st_size} bytes")


if __name__ == "__main__":
    main()
