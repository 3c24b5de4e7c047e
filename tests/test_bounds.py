"""Every global load and store of the decode kernels stays inside its buffer.

tp_selftest_decode_bounds (host code, no GPU) enumerates, for one launch,
each workgroup's, wave's and lane's memory accesses from the kernels' own
address functions (the ones decode_attention_kernel and fused_qk_kernel form
their pointers with), against buffers of the smallest sizes the C ABI admits:
page stores whose capacity equals the page count, the dense tail ending right
after the last row's valid tokens, the split-K workspace of
tp_decode_workspace_bytes.  The cases cover the unconditional-load idiom the
kernels rely on (a wave without a page loads its split's first page on lane
0's addresses; every lane loads scale dwords lane and lane + 64 of a page;
QJL sketches of whole token quads), 4- and 8-wave workgroups, one and two
combine tiers, tails, QJL, dense V, GQA from 1 to 20 and batch 2.  The
mutation cases plant the fault classes this idiom can hide and must fail.
"""

import ctypes

import pytest

from turbopolar_amd import _lib

LAYOUTS = {"default": (0, 4, 4, 64), "fast": (1, 4, 8, 0), "deep2": (0, 4, 2, 64), "l1_8bit": (0, 8, 4, 32)}


def run(layout="default", batch=1, hq=32, hkv=8, n_pages=64, capacity=None, tail=0, tail_stride=None, seq=None,
        pps=0, qjl=False, dense_v=False, kernel=0, mutate=0, qjl_bits=0):
    c = _lib.TPBoundsCase()
    c.batch, c.hq, c.hkv = batch, hq, hkv
    c.layout = _lib.make_layout(*LAYOUTS[layout])
    c.n_pages = n_pages
    c.capacity = n_pages if capacity is None else capacity
    c.tail_len = tail
    c.tail_stride = tail if tail_stride is None else tail_stride
    c.seq_len = n_pages * 64 + tail if seq is None else seq
    c.pages_per_split = pps
    c.qjl, c.qjl_capacity = int(qjl), n_pages
    c.dense_v, c.v_capacity = int(dense_v), n_pages
    c.kernel, c.mutate, c.qjl_bits = kernel, mutate, qjl_bits
    msg = ctypes.create_string_buffer(512)
    bad = _lib.lib().tp_selftest_decode_bounds(ctypes.byref(c), msg, 512)
    return bad, msg.value.decode()


CASES = [
    dict(),                                            # configs[0]-like: 4-page splits on 4 waves
    dict(n_pages=512),                                 # configs[2] at 32k: 16-page splits on 8 waves
    dict(n_pages=512, layout="fast"),
    dict(n_pages=3, pps=4),                            # waves without a page in every workgroup
    dict(n_pages=5, pps=8, layout="fast"),             # 8-page split on 4 waves, one wave without pages
    dict(n_pages=9, pps=16),                           # 8 waves, 16-page split, 7 waves without a second page
    dict(n_pages=17, pps=16, seq=7 * 64 + 3),          # pages past actual_seq_len: splits past the live pages
    dict(n_pages=64, tail=37, tail_stride=37),         # tail view ending its allocation
    dict(n_pages=64, tail=63, tail_stride=64, batch=2),
    dict(n_pages=40, tail=5, tail_stride=5, pps=1),    # one-page splits
    dict(hq=4, hkv=1, n_pages=2048, pps=8),            # two-tier combine (256 splits)
    dict(hq=8, hkv=1, n_pages=1030, pps=8),            # two tiers, ragged last group
    dict(hq=20, hkv=1, n_pages=33, pps=2),             # GQA 20: two head blocks
    dict(hq=12, hkv=2, n_pages=48, pps=3),             # GQA 6 on 4 waves
    dict(hq=64, hkv=8, n_pages=256),                   # configs[4] heads (GQA 8)
    dict(hq=8, hkv=8, n_pages=16),                     # GQA 1
    dict(n_pages=64, qjl=True),
    dict(n_pages=7, pps=4, qjl=True, layout="fast"),
    dict(n_pages=64, dense_v=True),
    dict(n_pages=3, pps=4, dense_v=True),
    dict(n_pages=20, layout="deep2", tail=9, tail_stride=9),
    dict(n_pages=20, layout="l1_8bit", pps=3),
    dict(n_pages=21, kernel=1),                        # fused QK: the last page reloaded past n_pages
    dict(n_pages=5, kernel=1, layout="fast"),
    dict(n_pages=5, kernel=1, layout="deep2", hq=20, hkv=1),
    dict(n_pages=100, capacity=128, batch=2, hq=16, hkv=4),
    dict(hq=24, hkv=2, n_pages=20, qjl=True),          # GQA 12: the row token order of default pages
    dict(hq=40, hkv=2, n_pages=9, pps=2, dense_v=True),
    dict(hq=8, hkv=2, n_pages=9, pps=2, qjl=True, tail=5, tail_stride=5),
    dict(n_pages=33, qjl=True, qjl_bits=40),           # QJL of any width: sketch dwords at byte offsets
    dict(hq=24, hkv=2, n_pages=7, pps=2, qjl=True, qjl_bits=8),
    dict(n_pages=5, pps=4, qjl=True, qjl_bits=256, layout="fast"),
    dict(hq=4, hkv=4, n_pages=3, qjl=True, qjl_bits=24, dense_v=True),
]


@pytest.mark.parametrize("case", CASES, ids=[",".join(f"{k}={v}" for k, v in c.items()) or "base" for c in CASES])
def test_decode_kernels_stay_in_bounds(case):
    bad, msg = run(**case)
    assert bad == 0, msg


@pytest.mark.parametrize("layout", ["default", "fast"])
def test_moved_v_scale_load_is_caught(layout):
    """Moving the second V-scale dword one page's scales (512 bytes) on reads
    past the last page of a store whose capacity equals its page count."""
    assert run(layout=layout, n_pages=16)[0] == 0
    bad, msg = run(layout=layout, n_pages=16, mutate=1)
    assert bad > 0 and "v_scales" in msg, msg


@pytest.mark.parametrize("case", [dict(n_pages=3, pps=4), dict(n_pages=5, pps=16, layout="fast"),
                                  dict(n_pages=5, pps=4, dense_v=True)])
def test_moved_no_page_load_is_caught(case):
    """A wave without a page of its own loads its split's first page; pointed
    at the next split's first page instead, the last split reads past the
    store."""
    assert run(**case)[0] == 0
    bad, msg = run(**case, mutate=2)
    assert bad > 0, msg


def test_bad_case_rejected():
    assert run(n_pages=8, capacity=4)[0] == 2 ** 64 - 1
