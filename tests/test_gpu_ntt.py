"""GPU parity of the batched NTT / INTT (C ABI pfa_ntt_forward / pfa_ntt_inverse)
against the CPU oracle: bit-exact residues on seeded uniform inputs and edge
values, for both arithmetic policies (primes < 2^50 run in FP64, larger ones in
64-bit integers), across every supported degree.

Mirrors the reference's test/ntt_test.cu (forward then inverse round trip on
N = 2^8..2^17, batch 1 and 10) and adds the known-answer comparison that test
lacks, plus a seeded sweep of random degrees, batch sizes, limb runs and
prime-size mixes."""
import numpy as np
import pytest

import py_oracle as O
from gpu_util import empty, first_mismatch, to_dev, to_host, uniform_limbs

pytestmark = pytest.mark.gpu


def make(N, bits, special=1):
    import pfa_native as P

    mods = O.create_coeff_modulus(N, bits)
    ctx = P.NativeContext(N, mods, special)
    orc = O.Oracle(N, mods, special)
    return mods, ctx, orc


@pytest.mark.parametrize("logn", [10, 11, 12, 13, 14, 15, 16, 17])
def test_ntt_fwd_inv_all_degrees(dev, logn):
    N = 1 << logn
    bits = [30, 40, 50, 60, 49, 58]
    mods, ctx, orc = make(N, bits)
    rng = np.random.default_rng(logn)
    M, L = 2, len(bits)
    x = uniform_limbs(rng, (M, L, N), mods)
    d = to_dev(x, dev)
    ctx.ntt_forward(d, M, L, 0)
    got = to_host(d)
    want = orc.ntt_fwd(x, threads=8)
    assert np.array_equal(got, want), first_mismatch(got, want)
    ctx.ntt_inverse(d, M, L, 0)
    back = to_host(d)
    assert np.array_equal(back, x), first_mismatch(back, x)
    # inverse of independent data against the oracle's inverse
    y = uniform_limbs(rng, (M, L, N), mods)
    dy = to_dev(y, dev)
    ctx.ntt_inverse(dy, M, L, 0)
    got = to_host(dy)
    want = orc.ntt_inv(y, threads=8)
    assert np.array_equal(got, want), first_mismatch(got, want)


def test_ntt_config1_cpu_case(dev):
    """benchmark config 1: N = 2^13, CoeffModulus::Create(8192, {50,50,55,60})."""
    N = 8192
    mods = O.create_coeff_modulus(N, [50, 50, 55, 60])
    import pfa_native as P

    ctx = P.NativeContext(N, mods, 1)
    orc = O.Oracle(N, mods, 1)
    rng = np.random.default_rng(0x5EED)
    x = uniform_limbs(rng, (1, 4, N), mods)
    d = to_dev(x, dev)
    ctx.ntt_forward(d, 1, 4, 0)
    want = orc.ntt_fwd(x)
    assert np.array_equal(to_host(d), want)
    ctx.ntt_inverse(d, 1, 4, 0)
    assert np.array_equal(to_host(d), x)


def test_ntt_config2_full_size(dev):
    """benchmark config 2: N = 2^16, 35 x 50-bit primes + one 60-bit special prime,
    batch of 2 polys x 35 limbs, bit-exact against the oracle."""
    N = 1 << 16
    mods, ctx, orc = make(N, [50] * 35 + [60])
    rng = np.random.default_rng(2)
    x = uniform_limbs(rng, (2, 35, N), mods)
    d = to_dev(x, dev)
    ctx.ntt_forward(d, 2, 35, 0)
    got = to_host(d)
    want = orc.ntt_fwd(x, threads=8)
    assert np.array_equal(got, want), first_mismatch(got, want)
    ctx.ntt_inverse(d, 2, 35, 0)
    assert np.array_equal(to_host(d), x)


def test_ntt_single_launch(dev, monkeypatch):
    """The single-launch NTT (opt-in with PFA_NTT_FLOW=1 at N = 2^16 for batches
    of 8+ limbs on a device that deals workgroups to 8 XCDs round-robin) against the oracle:
    both arithmetic policies in one batch, job counts that are and are not
    multiples of the XCD count, the smallest batch that takes it, and repeated
    launches (its control blocks alternate between calls)."""
    import pfa_native as P

    N = 1 << 16
    bits = [50, 60, 45, 50, 60, 50, 49, 58, 50, 60, 50]
    mods = O.create_coeff_modulus(N, bits + [60])
    monkeypatch.setenv("PFA_NTT_FLOW", "1")
    ctx = P.NativeContext(N, mods, 1)
    if not ctx.ntt_single_launch(2, 11):
        pytest.skip("this device does not deal workgroups to 8 XCDs round-robin; the two-launch NTT runs")
    assert not ctx.ntt_single_launch(1, 7)
    orc = O.Oracle(N, mods, 1)
    rng = np.random.default_rng(11)
    for M, L in [(2, 11), (3, 5), (1, 8), (4, 9), (2, 11)]:
        assert ctx.ntt_single_launch(M, L)
        x = uniform_limbs(rng, (M, L, N), mods)
        d = to_dev(x, dev)
        ctx.ntt_forward(d, M, L, 0)
        got = to_host(d)
        want = orc.ntt_fwd(x, threads=8)
        assert np.array_equal(got, want), (M, L, first_mismatch(got, want))
        ctx.ntt_inverse(d, M, L, 0)
        back = to_host(d)
        assert np.array_equal(back, x), (M, L, first_mismatch(back, x))
    ctx.synchronize()


def test_ntt_single_launch_expired_wait_is_an_error(dev, monkeypatch):
    """A single-launch NTT whose bounded wait gives up reports PFA_ERR_RUNTIME
    at the next synchronizing call instead of returning wrong residues.  The
    condition is forced from the host: a look-ahead window of one job makes most
    workgroups wait, and a wait bound of 0 ticks makes every such wait expire at
    its second poll; every workgroup then leaves and the kernel ends normally."""
    import pfa_native as P

    N = 1 << 16
    mods = O.create_coeff_modulus(N, [50] * 35 + [60])
    monkeypatch.setenv("PFA_NTT_FLOW", "1")
    monkeypatch.setenv("PFA_FLOW_WAIT_TICKS", "0")
    monkeypatch.setenv("PFA_FLOW_WINDOW", "1")
    ctx = P.NativeContext(N, mods, 1)
    if not ctx.ntt_single_launch(2, 35):
        pytest.skip("this device does not deal workgroups to 8 XCDs round-robin; the two-launch NTT runs")
    rng = np.random.default_rng(12)
    d = to_dev(uniform_limbs(rng, (2, 35, N), mods), dev)
    ctx.ntt_forward(d, 2, 35, 0)
    with pytest.raises(RuntimeError, match="single-launch NTT"):
        ctx.synchronize()
    # the record is cleared once reported
    ctx.synchronize()
    monkeypatch.delenv("PFA_FLOW_WAIT_TICKS")
    monkeypatch.delenv("PFA_FLOW_WINDOW")
    ok = P.NativeContext(N, mods, 1)
    x = uniform_limbs(rng, (2, 9, N), mods)
    d = to_dev(x, dev)
    ok.ntt_forward(d, 2, 9, 0)
    ok.ntt_inverse(d, 2, 9, 0)
    ok.synchronize()
    assert np.array_equal(to_host(d), x)


@pytest.mark.parametrize("logn,M,L", [(12, 2, 26), (16, 2, 25), (13, 4, 12)])
def test_ntt_large_batches_both_policies(dev, logn, M, L):
    """Batches of 48 limbs or more take the inverse rows pass with staged
    twiddles: forward and inverse against the oracle with 50- and 60-bit primes
    (FP64 and integer policies) mixed in one batch."""
    N = 1 << logn
    mods, ctx, orc = make(N, [50, 60] * (L // 2) + [50] * (L % 2) + [60])
    rng = np.random.default_rng(logn + M + L)
    x = uniform_limbs(rng, (M, L, N), mods)
    d = to_dev(x, dev)
    ctx.ntt_forward(d, M, L, 0)
    got, want = to_host(d), orc.ntt_fwd(x, threads=8)
    assert np.array_equal(got, want), first_mismatch(got, want)
    ctx.ntt_inverse(d, M, L, 0)
    back = to_host(d)
    assert np.array_equal(back, x), first_mismatch(back, x)


@pytest.mark.parametrize("fill", ["zero", "qm1", "one", "two"])
def test_ntt_edge_values(dev, fill):
    """Constant inputs (the reference's own all-1 / all-2 cases, test/ntt_test.cu:48-50,
    :103-106) and the extremes 0 and q-1 on both arithmetic policies."""
    N = 1 << 16
    mods, ctx, orc = make(N, [50, 60, 45, 60, 50])
    L = len(mods)
    x = np.zeros((1, L, N), dtype=np.uint64)
    for l, q in enumerate(mods):
        x[0, l] = {"zero": 0, "qm1": q - 1, "one": 1, "two": 2}[fill]
    d = to_dev(x, dev)
    ctx.ntt_forward(d, 1, L, 0)
    got = to_host(d)
    assert np.array_equal(got, orc.ntt_fwd(x))
    ctx.ntt_inverse(d, 1, L, 0)
    assert np.array_equal(to_host(d), x)


def test_ntt_start_offset_and_special_rows(dev):
    """start_modulus_idx: limbs use table rows start..start+L-1 (fntt_2d.cu:665-709)."""
    N = 1 << 12
    mods, ctx, orc = make(N, [50, 50, 60, 55, 60, 60], special=2)
    rng = np.random.default_rng(5)
    start, L = 2, 4
    x = uniform_limbs(rng, (3, L, N), mods[start:])
    d = to_dev(x, dev)
    ctx.ntt_forward(d, 3, L, start)
    assert np.array_equal(to_host(d), orc.ntt_fwd(x, start=start))


def test_ntt_argument_errors(dev):
    N = 1 << 12
    mods, ctx, orc = make(N, [50, 60])
    d = empty((1, 2, N), dev)
    with pytest.raises(ValueError):
        ctx.ntt_forward(d, 1, 3, 0)  # more limbs than primes
    with pytest.raises(ValueError):
        ctx.ntt_forward(d, 1, 2, 1)  # start + L beyond the table


def test_ntt_deterministic_across_calls(dev):
    """Same input, repeated launches -> identical residues (no races)."""
    N = 1 << 16
    mods, ctx, _ = make(N, [50] * 6 + [60])
    rng = np.random.default_rng(9)
    x = uniform_limbs(rng, (2, 6, N), mods)
    outs = []
    for _ in range(3):
        d = to_dev(x, dev)
        ctx.ntt_forward(d, 2, 6, 0)
        outs.append(to_host(d))
    assert all(np.array_equal(outs[0], o) for o in outs[1:])


def _ntt_shapes(n, seed):
    """(logn, M, L, start, bits): degree 2^10 .. 2^17, 1-4 polys, a run of L
    limbs starting at a random table row of a chain of random prime sizes."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        logn = int(rng.integers(10, 18))
        total = int(rng.integers(2, 13))
        bits = [int(b) for b in rng.choice([30, 36, 40, 45, 49, 50, 55, 58, 60], size=total)]
        start = int(rng.integers(0, total))
        L = int(rng.integers(1, total - start + 1))
        M = int(rng.integers(1, 5)) if logn < 17 else 1
        out.append((logn, M, L, start, bits))
    return out


@pytest.mark.parametrize("logn,M,L,start,bits", _ntt_shapes(10, 77))
def test_ntt_random_shapes(dev, logn, M, L, start, bits):
    """Seeded random degrees, batch sizes, limb runs and prime-size mixes:
    forward against the oracle, inverse back to the input, bit for bit."""
    N = 1 << logn
    mods, ctx, orc = make(N, bits)
    rng = np.random.default_rng(logn * 100 + L)
    x = uniform_limbs(rng, (M, L, N), mods[start:start + L])
    d = to_dev(x, dev)
    ctx.ntt_forward(d, M, L, start)
    got = to_host(d)
    want = orc.ntt_fwd(x, start=start, threads=8)
    assert np.array_equal(got, want), first_mismatch(got, want)
    ctx.ntt_inverse(d, M, L, start)
    back = to_host(d)
    assert np.array_equal(back, x), first_mismatch(back, x)
