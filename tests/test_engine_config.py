"""ckks_engine's configuration checks (src/ckks_engine.cu:62-91), which run
before anything touches the GPU: the same conditions and exception classes as
the reference's binding (std::invalid_argument -> ValueError)."""
import pytest

import pyPhantom as ph


def _cfg(**kw):
    c = ph.ckks_engine_config()
    for k, v in kw.items():
        setattr(c, k, v)
    return c


def test_config_defaults():
    """CKKSEngineConfig's defaults (include/ckks_engine.h:29-95)."""
    c = ph.ckks_engine_config()
    assert (c.log_n, c.user_scale, c.num_scale_levels, c.sparse_hw, c.num_special_primes) == (16, 2.0 ** 40, 14, 128, 6)
    assert c.include_user_rotations and not c.split_scale_down
    assert c.user_rotation_steps == [] and c.user_rotation_target_chain_indices == []
    assert not c.build_two_scale_arrays and not c.use_bootstrap_to_17_levels
    # the default chain: 1 + 14 + 3 + 9 + 3 = 30 primes, 30 % 6 == 0
    assert len(ph.ckks_engine_coeff_bits(c.num_scale_levels, c.num_special_primes)) == 30 + 6


@pytest.mark.parametrize("kw,msg", [
    (dict(log_n=15), "pins log_n=16"),
    (dict(num_scale_levels=1), "num_scale_levels must be >= 2"),
    (dict(num_special_primes=0), "num_special_primes must be >= 1"),
    (dict(num_scale_levels=15), "divisible by num_special_primes"),       # size_Q 31
    (dict(use_bootstrap_to_17_levels=True), "divisible by num_special_primes"),  # 14 + 14 = 28
])
def test_config_errors(kw, msg):
    with pytest.raises(ValueError, match=msg):
        ph.ckks_engine(_cfg(**kw))
