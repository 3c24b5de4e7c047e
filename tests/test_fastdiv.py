"""The decode kernel's workgroup-index division by launch constants
(multiply and shift with host-computed constants, Granlund and Montgomery
theorem 4.2), checked inside the library on the host against integer
division.  No GPU needed."""
import ctypes

from turbopolar_amd import _lib


def test_fastdiv_matches_integer_division():
    L = _lib.lib()
    checks = ctypes.c_ulonglong(0)
    bad = L.tp_selftest_fastdiv(4096, ctypes.byref(checks))
    assert bad == 0
    assert checks.value > 4096 * 700  # every divisor: range ends, multiples across the range, small dividends
