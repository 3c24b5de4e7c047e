"""The C-ABI library loads, exports every symbol include/turbopolar.h declares,
and validates its arguments on the host (no GPU needed for these paths)."""

import ctypes
import re

import pytest

from turbopolar_amd import _lib
from turbopolar_amd.payload import packed_row_bytes


def test_library_exports_every_header_symbol():
    syms = _lib.header_symbols()
    assert len(syms) >= 12
    handle = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [s for s in syms if not hasattr(handle, s)]
    assert not missing, missing
    # and the binding declares a signature for each of them
    assert sorted(_lib._SIGNATURES) == syms


def test_header_declares_c_linkage_only():
    text = _lib.HEADER_PATH.read_text()
    assert 'extern "C"' in text
    assert "torch" not in text.lower() and "hipStream_t" not in text


def test_version_and_last_error():
    L = _lib.lib()
    assert L.tp_version() == 100
    assert isinstance(L.tp_last_error(), bytes)


@pytest.mark.parametrize("l1,deep,split", [(4, 4, 64), (4, 8, 0), (8, 2, 32), (4, 2, 46), (8, 4, 128), (4, 4, 2)])
def test_row_bytes_match_packing_rule(l1, deep, split):
    layout = _lib.make_layout(False, l1, deep, split)
    assert _lib.row_bytes(layout) == (packed_row_bytes(split // 2, l1), packed_row_bytes(64 - split // 2, deep))


@pytest.mark.parametrize("l1,deep,split,msg", [
    (3, 4, 64, "k_angle_bits_level1"),
    (4, 3, 64, "k_angle_bits_deep"),
    (4, 4, 63, "split_dim"),
    (4, 4, 130, "split_dim"),
])
def test_layout_rejections(l1, deep, split, msg):
    with pytest.raises(ValueError, match=msg):
        _lib.row_bytes(_lib.make_layout(False, l1, deep, split))


def _fake_pages(capacity=8):
    # Aligned, never dereferenced: validation fails before any device access.
    return _lib.TPPages(4096, 8192, 12288, 16384, 20480, 24576, capacity)


def test_encode_argument_validation():
    L = _lib.lib()
    lay = _lib.make_layout(False, 4, 4, 64)
    pages = _fake_pages()
    st = L.tp_encode_pages(4096, 8192, 2, 1, 64, 0, 64, ctypes.byref(lay), ctypes.byref(pages), 0, None)
    assert st == _lib.TP_ERR_INVALID and b"in_dtype" in L.tp_last_error()
    st = L.tp_encode_pages(4096, 8192, 0, 1, 64, 10, 64, ctypes.byref(lay), ctypes.byref(pages), 0, None)
    assert st == _lib.TP_ERR_INVALID and b"token range" in L.tp_last_error()
    st = L.tp_encode_pages(4096, 8192, 0, 1, 64 * 20, 0, 64 * 9, ctypes.byref(lay), ctypes.byref(pages), 0, None)
    assert st == _lib.TP_ERR_INVALID and b"capacity" in L.tp_last_error()
    st = L.tp_encode_pages(4100, 8192, 0, 1, 64, 0, 64, ctypes.byref(lay), ctypes.byref(pages), 0, None)
    assert st == _lib.TP_ERR_INVALID and b"aligned" in L.tp_last_error()
    assert L.tp_encode_pages(4096, 8192, 0, 1, 64, 0, 0, ctypes.byref(lay), ctypes.byref(pages), 0, None) == 0


def test_decode_pages_gather_argument_validation():
    """tp_decode_pages_gather (fetch_blocks' one launch) rejects a missing
    index array, a stored-page count outside the capacity, a misaligned index
    array and a bad output before any device access; no indices is a no-op."""
    L = _lib.lib()
    lay = _lib.make_layout(False, 4, 4, 64)
    pages = _fake_pages(capacity=8)
    g = L.tp_decode_pages_gather
    assert g(ctypes.byref(lay), ctypes.byref(pages), 2, 4, None, 3, 4096, None, None) == _lib.TP_ERR_INVALID
    assert b"index array" in L.tp_last_error()
    for n_stored in (0, 9):
        assert g(ctypes.byref(lay), ctypes.byref(pages), 2, n_stored, 4096, 3, 4096, None, None) == _lib.TP_ERR_INVALID
        assert b"bad page range" in L.tp_last_error()
    assert g(ctypes.byref(lay), ctypes.byref(pages), 2, 4, 4098, 3, 4096, None, None) == _lib.TP_ERR_INVALID
    assert g(ctypes.byref(lay), ctypes.byref(pages), 2, 4, 4096, 3, 4100, None, None) == _lib.TP_ERR_INVALID
    assert g(ctypes.byref(lay), ctypes.byref(pages), 2, 4, None, 0, None, None, None) == _lib.TP_OK


def test_decode_attention_argument_validation():
    L = _lib.lib()
    lay = _lib.make_layout(False, 4, 4, 64)
    pages = _fake_pages()

    def call(**kw):
        a = dict(q=4096, batch=1, hq=8, hkv=2, n_pages=4, tk=None, tv=None, tail=0, tstride=0, seq=256,
                 pps=0, ws=None, wsb=0, out=8192)
        a.update(kw)
        st = L.tp_decode_attention(a["q"], a["batch"], a["hq"], a["hkv"], ctypes.byref(lay), ctypes.byref(pages),
                                   a["n_pages"], a["tk"], a["tv"], a["tail"], a["tstride"], a["seq"], 0.088, a["pps"],
                                   a["ws"], a["wsb"], a["out"], None)
        return st, L.tp_last_error().decode()

    assert call(hq=7)[0] == _lib.TP_ERR_INVALID
    assert call(n_pages=9)[0] == _lib.TP_ERR_INVALID
    st, msg = call(tail=64, tk=4096, tv=4096, tstride=64)
    assert st == _lib.TP_ERR_INVALID and "tail_len" in msg
    # A length past the stored tokens is accepted (the reference only masks
    # tokens at or past it); pps=1 without a workspace then stops the call at
    # the workspace check, before any launch.
    st, msg = call(seq=10**9, pps=1)
    assert st == _lib.TP_ERR_WORKSPACE and "workspace" in msg
    st, msg = call(seq=0)
    assert st == _lib.TP_ERR_INVALID and "actual_seq_len" in msg
    st, msg = call(n_pages=0)
    assert st == _lib.TP_ERR_INVALID and "nothing to attend" in msg
    st, msg = call(pps=1)  # 4 splits need a workspace
    assert st == _lib.TP_ERR_WORKSPACE and "workspace" in msg
    # The grid is (hkv, batch x head blocks, splits), at most 65535 splits:
    # 2^30 one-page splits of 8 kv heads do not fit, nor do 65536.
    big = _fake_pages(capacity=1 << 30)
    st = L.tp_decode_attention(4096, 1, 8, 8, ctypes.byref(lay), ctypes.byref(big), 1 << 30, None, None, 0, 0,
                               (1 << 30) * 64, 0.088, 1, None, 0, 8192, None)
    assert st == _lib.TP_ERR_INVALID and b"grid limit" in L.tp_last_error()
    st = L.tp_decode_attention(4096, 1, 8, 8, ctypes.byref(lay), ctypes.byref(big), 65536, None, None, 0, 0,
                               65536 * 64, 0.088, 1, None, 0, 8192, None)
    assert st == _lib.TP_ERR_INVALID and b"grid limit" in L.tp_last_error()
    st = L.tp_decode_attention(4096, 1, 8, 2, ctypes.byref(lay), ctypes.byref(big), 1537, None, None, 0, 0,
                               1537 * 64, 0.088, 1, None, 0, 8192, None)
    assert st == _lib.TP_ERR_WORKSPACE  # any number of splits that fits the grid is accepted


def test_decode_attention_dense_v_argument_validation():
    """tp_decode_attention_dense_v: dense V is required, 16-byte aligned and
    at least n_pages deep; the page structure's V fields are not needed.
    Every rejected call returns before any device access."""
    L = _lib.lib()
    lay = _lib.make_layout(False, 4, 4, 64)
    pages = _lib.TPPages(4096, 8192, 12288, 16384, None, None, 8)

    def call(**kw):
        a = dict(n_pages=4, v=32768, vcap=4, seq=256, pps=0)
        a.update(kw)
        st = L.tp_decode_attention_dense_v(4096, 1, 8, 2, ctypes.byref(lay), ctypes.byref(pages), a["n_pages"],
                                           None, a["v"], a["vcap"], a["seq"], 0.088, a["pps"], None, 0, 8192, None)
        return st, L.tp_last_error().decode()

    assert call(v=None)[0] == _lib.TP_ERR_INVALID
    assert call(n_pages=0)[0] == _lib.TP_ERR_INVALID
    st, msg = call(vcap=3)
    assert st == _lib.TP_ERR_INVALID and "v_capacity" in msg
    st, msg = call(v=32770)
    assert st == _lib.TP_ERR_INVALID and "aligned" in msg
    assert call(seq=0)[0] == _lib.TP_ERR_INVALID
    # Valid arguments with NULL V codes and scales reach the workspace check
    # (4 one-page splits need one), still before any launch.
    st, msg = call(pps=1)
    assert st == _lib.TP_ERR_WORKSPACE and "workspace" in msg


def test_workspace_sizes():
    L = _lib.lib()
    # Llama-3-8B shape at 32k: one workgroup per CU -> 16 pages per split
    assert L.tp_default_pages_per_split(1, 32, 8, 512) == 16
    n = L.tp_decode_workspace_bytes(1, 32, 8, 512, 0, 16)
    counters = L.tp_decode_counter_bytes(1, 32, 8)
    assert counters == 65536  # fixed area: records start at the same offset for every shape
    splits = 32
    # (m, l) rows in fp32, the splits' normalised outputs in fp16
    assert n == counters + 8 * splits * 16 * 2 * 4 + 8 * splits * 16 * 128 * 2
    # GQA group > 16 uses two head blocks
    assert L.tp_decode_counter_bytes(2, 40, 2) == 65536
    assert L.tp_decode_counter_bytes(4096, 8, 8) == 32768 * 4  # beyond 16384 units the area grows
    assert L.tp_decode_workspace_bytes(1, 40, 2, 2, 0, 1) > L.tp_decode_workspace_bytes(1, 16, 1, 2, 0, 1)


def test_product_has_no_oracle_dependency():
    """The product package never imports the oracle (the oracle checks it)."""
    import pathlib

    pkg = pathlib.Path(_lib.__file__).parent
    for f in pkg.glob("*.py"):
        src = f.read_text()
        assert not re.search(r"^\s*(import|from)\s+oracle\b", src, re.M), f


def test_append_stage_argument_validation():
    L = _lib.lib()
    args = dict(k=4096, v=8192, dt=0, bh=8, tok=1, cb=0, n=1, tk=12288, tv=16384, tt=64, tp=0)

    def call(check, flag):
        a = args
        st = L.tp_append_stage(a["k"], a["v"], a["dt"], a["bh"], a["tok"], a["cb"], a["n"], a["tk"], a["tv"],
                               a["tt"], a["tp"], check, flag, 1, None)
        return st, L.tp_last_error().decode()

    for check in (-1, 3):
        st, msg = call(check, 20480)
        assert st == _lib.TP_ERR_INVALID and "check must be" in msg
    for check in (1, 2):
        st, msg = call(check, None)
        assert st == _lib.TP_ERR_INVALID and "flag" in msg
    L.tp_append_stage(4096, 8192, 0, 8, 1, 0, 1, 12288, 16384, 64, 0, 2, 20480, 3, None)
    assert "even epoch" in L.tp_last_error().decode()  # check 2 takes even epochs


def test_integration_stub_matches_the_binding(monkeypatch):
    """The ctypes stub that INTEGRATION.md offers to the reference declares the
    same signatures and struct layouts as the package's own binding."""
    import pathlib

    doc = (pathlib.Path(_lib.__file__).parent.parent / "INTEGRATION.md").read_text()
    blocks = re.findall(r"```python\n(.*?)```", doc, re.S)
    stub = next(b for b in blocks if "class TPPages" in b)
    real_cdll = ctypes.CDLL
    monkeypatch.setattr(ctypes, "CDLL", lambda name, *a, **k: real_cdll(str(_lib.LIB_PATH), *a, **k))
    ns = {}
    exec(compile(stub, "INTEGRATION.md", "exec"), ns)
    for struct_name in ("TPPageLayout", "TPPages"):
        mine, theirs = getattr(_lib, struct_name), ns[struct_name]
        assert [(n, t) for n, t in theirs._fields_] == [(n, t) for n, t in mine._fields_]
        assert ctypes.sizeof(theirs) == ctypes.sizeof(mine)
    for name in ("tp_decode_attention", "tp_decode_workspace_bytes"):
        fn = getattr(ns["_lib"], name)
        restype, argtypes = _lib._SIGNATURES[name]
        assert fn.restype == restype
        norm = [getattr(t, "_type_", t).__name__ if t.__name__.startswith("LP_") else t.__name__ for t in fn.argtypes]
        want = [getattr(t, "_type_", t).__name__ if t.__name__.startswith("LP_") else t.__name__ for t in argtypes]
        norm = ["tp_page_layout" if n == "TPPageLayout" else "tp_pages" if n == "TPPages" else n for n in norm]
        want = ["tp_page_layout" if n == "TPPageLayout" else "tp_pages" if n == "TPPages" else n for n in want]
        assert norm == want, name


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    """Without the built library every kernel call raises; nothing falls back to the CPU."""
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libturbopolar_hip.so")
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="not built.*no CPU fallback"):
        _lib.lib()
