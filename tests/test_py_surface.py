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


def test_binding_names_present():
    """Every class, enum and function name the reference's module binds for
    the CKKS path is importable here (binding.cu:31-590; the LLM blocks and
    BFV's batch_encoder are outside this core)."""
    names = ["scheme_type", "mul_tech_type", "sec_level_type", "modulus", "create_coeff_modulus",
             "create_plain_modulus", "params", "cuda_stream", "context", "secret_key", "public_key", "relin_key",
             "galois_key", "get_elt_from_step", "get_elts_from_steps", "ckks_encoder", "plaintext", "ciphertext",
             "negate", "add", "add_plain", "add_many", "sub", "sub_plain", "multiply", "multiply_and_relin",
             "multiply_plain", "relinearize", "rescale_to_next", "mod_switch_to_next", "mod_switch_to",
             "mod_switch_to_inplace", "apply_galois", "rotate", "apply_galois_with_key", "rotate_with_key",
             "hoisting", "hoist_rotations", "small_bootstrap_key", "bootstrap_key", "bootstrap_required_galois_elts",
             "create_bootstrap_key", "bootstrap", "ckks_engine_config", "ckks_engine", "set_cuda_device",
             "get_cuda_device_count", "single_chain_plaintext", "encode_single_chain_plaintext", "scp_from_bytes",
             "expand_single_chain_to_full", "inner_sum", "replicate", "bsgs_diagonals", "pre_encode_bsgs_diagonals",
             "bsgs_required_steps", "bsgs_matmul_preencoded", "compute_bsgs_babies", "bsgs_apply_giants_with_babies",
             "complex_fold_mode", "pre_encode_bsgs_diagonals_complex", "eval_polynomial", "complex_bsgs_diagonals",
             "bsgs_apply_giants_with_babies_complex"]
    assert [n for n in names if not hasattr(ph, n)] == []
    assert [m.name for m in ph.complex_fold_mode] == ["Rows", "ColsConj"]


def test_cuda_stream_needs_a_device():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a device is visible; the GPU tests cover cuda_stream")
    with pytest.raises(RuntimeError):
        ph.cuda_stream()


def test_stream_handle_maps_torch_default_stream():
    """torch's default stream (handle 0) goes to the library as hipStreamLegacy
    (1), not as NULL, which the C ABI reads as hipStreamPerThread; any other
    stream's handle passes through."""
    import pfa_native as P

    class S:
        def __init__(self, h):
            self.cuda_stream = h

    assert P.stream_handle(S(0)) == P.HIP_STREAM_LEGACY == 1
    assert P.stream_handle(S(0x5A5A0)) == 0x5A5A0
