"""CPU-side checks of the C ABI (no GPU needed): libphantom_amd.so loads, exports
every symbol declared in include/phantom_amd.h, and its host logic (modulus
generation, Galois elements, argument validation and error mapping) agrees
with the oracle and with the reference's documented behaviour."""
import os
import re

import pytest

import py_oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    names = set()
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if fn.endswith(".h"):
            text = open(os.path.join(ROOT, "include", fn)).read()
            names |= set(re.findall(r"\b(pfa_\w+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    import pfa_native as P

    lib = P.lib()
    names = header_symbols()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # the Python binding table covers the whole header, one to one
    assert sorted(P.SIGNATURES) == names


def test_abi_version():
    import pfa_native as P

    assert P.lib().pfa_abi_version() == 1


@pytest.mark.parametrize("N,bits", [
    (8192, [50, 50, 55, 60]),
    (65536, [50] * 35 + [60]),
    (65536, [60] + [50] * 23 + [60] * 4),
    (1024, [30, 30, 40, 20]),
])
def test_create_coeff_modulus_matches_oracle(N, bits):
    import pfa_native as P

    assert P.create_coeff_modulus(N, bits) == O.create_coeff_modulus(N, bits)


def test_create_coeff_modulus_errors():
    import pfa_native as P

    with pytest.raises(ValueError):
        P.create_coeff_modulus(8192, [61])  # above the 60-bit limit
    with pytest.raises(ValueError):
        P.create_coeff_modulus(1000, [50])  # degree not a power of two
    with pytest.raises(ValueError):
        P.create_coeff_modulus(1 << 18, [50])  # degree above 2^17
    with pytest.raises(ValueError):
        P.create_coeff_modulus(1 << 12, [40] * 65)  # more than 64 moduli
    assert len(P.create_coeff_modulus(1 << 12, [40] * 64)) == 64
    with pytest.raises(RuntimeError):
        P.create_coeff_modulus(1 << 16, [18])  # no 18-bit prime = 1 mod 2^17
    assert "prime" in P.lib().pfa_last_error().decode()


@pytest.mark.parametrize("N", [1024, 8192, 65536])
def test_galois_elt_matches_oracle(N):
    import pfa_native as P

    for step in (0, 1, -1, 2, 5, -7, N // 2 - 1, -(N // 2 - 1)):
        assert P.galois_elt_from_step(step, N) == O.elt_from_step(step, N)
    with pytest.raises(ValueError):
        P.galois_elt_from_step(N // 2, N)  # "step count too large" (include/galois.cuh:29-31)


def test_null_context_is_an_error():
    import ctypes as C

    import pfa_native as P

    rc = P.lib().pfa_ntt_forward(None, None, 1, 1, 0, None)
    assert rc == P.PFA_ERR_INVALID_ARGUMENT
    assert "null context" in P.lib().pfa_last_error().decode()
    rc = P.lib().pfa_rescale(None, 1, None, 2, None, None)
    assert rc == P.PFA_ERR_INVALID_ARGUMENT
    out = C.c_void_p()
    # moduli that are not = 1 mod 2N are rejected before any device work
    bad = (C.c_uint64 * 2)(97, 193)
    rc = P.lib().pfa_context_create(1024, bad, 2, 1, 0, C.byref(out))
    assert rc == P.PFA_ERR_INVALID_ARGUMENT


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU; --gpus N > 1 exits with a message (no GPU needed)."""
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
