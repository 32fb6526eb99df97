"""The small value types of the reference's Python module (python/src/binding.cu:
46-70): sec_level_type, modulus, create_coeff_modulus / create_plain_modulus
and cuda_stream.  None of these launches a kernel, so they run on the CPU."""
import pytest

import py_oracle as O
import pyPhantom as ph


def test_sec_level_type_values():
    assert [int(v) for v in ph.sec_level_type] == [0, 128, 192, 256]
    assert ph.sec_level_type.tc128.name == "tc128"


def test_modulus_value_and_limits():
    """src/host/modulus.cu:15-24: zero is allowed, 1 and values of more than
    61 bits are rejected with std::invalid_argument (ValueError here)."""
    p = ph.modulus((1 << 61) - 1)
    assert p.value == (1 << 61) - 1 and p.bit_count() == 61 and not p.is_zero()
    assert ph.modulus(0).is_zero() and ph.modulus().value == 0
    for bad in (1, 1 << 61, -5):
        with pytest.raises(ValueError):
            ph.modulus(bad)


@pytest.mark.parametrize("N,bits", [(1 << 12, [60, 40, 40, 60]), (1 << 16, [60] + [50] * 6 + [60] * 2)])
def test_create_coeff_modulus_gives_moduli(N, bits):
    mods = ph.create_coeff_modulus(N, bits)
    assert all(isinstance(m, ph.modulus) for m in mods)
    assert [m.value for m in mods] == O.create_coeff_modulus(N, bits)
    assert all(m.value % (2 * N) == 1 and m.bit_count() == b for m, b in zip(mods, bits))
    # a list of moduli sets the parameters as the reference's vector<Modulus> does
    p = ph.params(ph.scheme_type.ckks)
    p.set_coeff_modulus(mods)
    assert p.coeff_modulus == O.create_coeff_modulus(N, bits)
    assert all(type(m) is int for m in p.coeff_modulus)


def test_create_plain_modulus_and_ckks_rejection():
    t = ph.create_plain_modulus(1 << 13, 20)
    assert isinstance(t, ph.modulus) and t.bit_count() == 20 and t.value % (1 << 14) == 1
    with pytest.raises(ValueError):
        ph.params(ph.scheme_type.ckks).set_plain_modulus(t)


def test_cuda_stream_needs_a_device():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a device is visible; the GPU tests cover cuda_stream")
    with pytest.raises(RuntimeError):
        ph.cuda_stream()
