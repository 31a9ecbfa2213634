"""The device division shortcut (a refined reciprocal shared by every quotient with
the same divisor) returns the compiler's IEEE float32 quotient bit for bit inside its
operand range: random signs, exponents in [-40, 40) and mantissas, zero numerators
and the range's end values (cp_check_division)."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", [0, 1 << 40, 12345678901])
def test_shared_divisor_quotient_is_ieee(seed):
    from perm_amd import _lib
    lib = _lib.load()
    bad = ctypes.c_int64(-1)
    n = 1 << 28
    print(f"division check seed={seed} n={n}", flush=True)
    rc = lib.cp_check_division(n, seed, ctypes.byref(bad),
                               ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, lib.cp_last_error()
    assert bad.value == 0, f"{bad.value} of {n} quotients differ"
