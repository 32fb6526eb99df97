"""Benchmark of the MI355X CKKS hot path (one JSON line on stdout).

Headline (the project metric, config 2): batched forward negacyclic NTT at
N = 2^16 over a batch of 2 polys x 35 limbs (35 x 50-bit primes; the 60-bit
special prime is in the table but not transformed).  One step = one forward
NTT of one batch, inputs resident in HBM.  value = limbs transformed per second.

To keep the measurement an HBM measurement, the timed steps cycle through
several distinct batches whose total size exceeds the 256 MiB Infinity Cache,
so no step finds its batch cached from the previous one.

Also reported (same line): inverse NTT limbs/s, HMult + relinearize + rescale
latency for config 3 (|Q| = 24, alpha = 4, dnum = 6) and for the metric's
"L=35" variant (|Q| = 35, alpha = 1), and the config-4 BSGS matrix-vector
product (4096 x 4096 matrix, 64 baby x 64 giant steps, L = 20) and the
config-5 bootstrap (latency and refreshed precision bits).

cpu_baseline: the CPU oracle's forward NTT (oracle/ckks_oracle.c, a C
restatement of the reference algorithm) on the same workload, single thread,
timed on this host for a bounded sample.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "phantom-fhe_amd"), os.path.join(ROOT, "oracle")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

N = 1 << 16
LIMBS = 35
POLYS = 2
HBM_PEAK_GBS = 8000.0
LIMB_BYTES = N * 8
# algorithmic bytes of one forward NTT of the batch: each residue read once and written once
NTT_BYTES = POLYS * LIMBS * N * 16


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def uniform(torch, shape, mods, dev, gen):
    """uint64 residues uniform in [0, q_l) on the device; limb axis is -2."""
    *pre, L, n = shape
    out = torch.empty(tuple(shape), dtype=torch.int64, device=dev)
    for l in range(L):
        out[..., l, :] = torch.randint(0, int(mods[l]), tuple(pre) + (n,), dtype=torch.int64, device=dev,
                                       generator=gen)
    return out.view(torch.uint64)


def spin_up(torch, step, ms=40.0, chunk=20, cap=20000):
    """Runs step(i) untimed until the GPU has been kept busy for about `ms`
    milliseconds, before a workload's warm-up and timed steps: the MI355X's
    clocks ramp up under sustained load (measured on the config-2 forward NTT:
    36.9-37.4 us per transform after 20 warm-up steps, 33.9-34.2 us after 500
    or 2000, interleaved on one box).  Returns the number of steps run."""
    torch.cuda.synchronize()
    t0, n = time.perf_counter(), 0
    while (time.perf_counter() - t0) * 1e3 < ms and n < cap:
        for _ in range(chunk):
            step(n)
            n += 1
        torch.cuda.synchronize()
    return n


def time_ntt(torch, ctx, batches, steps, warmup, inverse=False):
    """Returns (wall seconds for `steps` transforms, average ms per transform from
    HIP events recorded on the launch stream around the whole timed region)."""
    import pfa_native as P

    stream = torch.cuda.current_stream()
    h = P.stream_handle(stream)
    fn = ctx.ntt_inverse if inverse else ctx.ntt_forward
    spin_up(torch, lambda i: fn(batches[i % len(batches)], POLYS, LIMBS, 0, h))
    for i in range(warmup):
        fn(batches[i % len(batches)], POLYS, LIMBS, 0, h)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(steps):
        fn(batches[i % len(batches)], POLYS, LIMBS, 0, h)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall, e0.elapsed_time(e1) / steps


def time_copy(torch, P, batches, steps, warmup):
    """The hand-written streaming copy (pfa_stream_copy: 16-byte nontemporal
    loads and stores) of the same 2 x 35-limb batches, rotating sources and
    destinations: the achievable one-read-one-write rate the NTT's 73.4 MB per
    transform is measured against.  Returns microseconds per copy (HIP events)."""
    stream = torch.cuda.current_stream()
    h = P.stream_handle(stream)
    dsts = [torch.empty_like(b) for b in batches]
    n = len(batches)
    spin_up(torch, lambda i: P.stream_copy(dsts[(i + 3) % n], batches[i % n], 0, h))
    for i in range(warmup):
        P.stream_copy(dsts[(i + 3) % n], batches[i % n], 0, h)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for i in range(steps):
        P.stream_copy(dsts[(i + 3) % n], batches[i % n], 0, h)
    e1.record(stream)
    torch.cuda.synchronize()
    del dsts
    return e0.elapsed_time(e1) / steps * 1e3


def ntt_limb_sweep(torch, P, dev, gen, steps):
    """Forward and inverse NTT time (HIP events, 10 rotating batches) for 2 polys
    x L limbs of 50-bit primes at N = 2^16, over L around the config-2 batch.
    Both passes process 16 tiles per limb on 4 x #CU resident workgroups, so the
    sweep shows what a batch whose tile count exceeds the resident workgroups by
    a little pays for its second round."""
    mods = P.create_coeff_modulus(N, [50] * 48 + [60])
    ctx = P.NativeContext(N, mods, 1)
    stream = torch.cuda.current_stream()
    h = P.stream_handle(stream)
    rows = []
    for L in (28, 30, 32, 33, 34, 35, 36, 40, 48):
        bs = [uniform(torch, (POLYS, L, N), mods, dev, gen) for _ in range(10)]
        us = []
        for fn in (ctx.ntt_forward, ctx.ntt_inverse):
            for i in range(20):
                fn(bs[i % 10], POLYS, L, 0, h)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            e0.record(stream)
            for i in range(steps):
                fn(bs[i % 10], POLYS, L, 0, h)
            e1.record(stream)
            torch.cuda.synchronize()
            us.append(e0.elapsed_time(e1) / steps * 1000)
        rows.append({"limbs": POLYS * L, "tiles_per_pass": POLYS * L * 16, "forward_us": round(us[0], 2),
                     "inverse_us": round(us[1], 2)})
        log(f"bench: sweep {POLYS * L} limbs: forward {us[0]:.2f} us, inverse {us[1]:.2f} us")
        del bs
    return rows


def time_hmult(torch, P, dev, gen, nq, alpha, steps, warmup):
    """multiply_and_relin + rescale on fresh chain-index-1 ciphertexts; returns ms per op."""
    bits = [60] + [50] * (nq - 1) + [60] * alpha
    mods = P.create_coeff_modulus(N, bits)
    ctx = P.NativeContext(N, mods, alpha)
    dnum = nq // alpha
    a = uniform(torch, (2, nq, N), mods, dev, gen)
    b = uniform(torch, (2, nq, N), mods, dev, gen)
    key = torch.empty((dnum, 2, nq + alpha, N), dtype=torch.uint64, device=dev)
    for d in range(dnum):
        key[d] = uniform(torch, (2, nq + alpha, N), mods, dev, gen)
    out = torch.empty((2, nq, N), dtype=torch.uint64, device=dev)
    res = torch.empty((2, nq - 1, N), dtype=torch.uint64, device=dev)
    s = P.stream_handle(torch.cuda.current_stream())

    def separate(_):
        ctx.multiply_and_relin(1, a, b, key, out, s)
        ctx.rescale(1, out, res, s)

    spin_up(torch, separate, chunk=4)
    for i in range(warmup):
        separate(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        ctx.multiply_and_relin(1, a, b, key, out, s)
        ctx.rescale(1, out, res, s)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    # the same operation as one call (pfa_multiply_relin_rescale), checked equal
    fused = torch.empty_like(res)
    for _ in range(warmup):
        ctx.multiply_relin_rescale(1, a, b, key, fused, s)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(steps):
        ctx.multiply_relin_rescale(1, a, b, key, fused, s)
    e1.record()
    torch.cuda.synchronize()
    fused_ms = e0.elapsed_time(e1) / steps
    if not torch.equal(fused, res):
        raise RuntimeError("fused multiply_relin_rescale differs from multiply_and_relin + rescale")
    compulsory = (2 * 2 * nq + dnum * 2 * (nq + alpha) + 2 * (nq - 1)) * LIMB_BYTES
    del key, a, b, out, res, fused
    ctx.close()
    best = min(ms, fused_ms)
    return {"ms": round(best, 4), "separate_calls_ms": round(ms, 4), "fused_call_ms": round(fused_ms, 4),
            "compulsory_bytes": compulsory,
            "hbm_roofline_frac": round(compulsory / (best * 1e-3) / (HBM_PEAK_GBS * 1e9), 4),
            "chain": f"{{60, 50 x {nq - 1}, 60 x {alpha}}}", "dnum": dnum}


def time_bsgs(torch, steps, warmup):
    """benchmark config 4 through the pyPhantom API: y = W x for a 4096 x 4096
    matrix uniform in [-1/64, 1/64] (seeded), x uniform in [-1, 1] replicated over
    the 2^15 slots with period 4096, baby 64 / giant 64, L = 20 (chain
    {60, 40 x 19, 60 x 4}), scale 2^40, sparse ternary secret h = 192.  Times the
    whole product (63 baby rotations, the giants' accumulation, 63 giant
    rotations, the rescale) with the expanded diagonals resident; the one-time
    encode and expansion are reported separately, and the decrypted result is
    checked against numpy."""
    import numpy as np

    import pyPhantom as ph

    d_pad, M = 4096, 64
    p = ph.params(ph.scheme_type.ckks)
    p.set_poly_modulus_degree(N)
    p.set_coeff_modulus(ph.create_coeff_modulus(N, [60] + [40] * 19 + [60] * 4))
    p.set_special_modulus_size(4)
    p.set_galois_elts(ph.get_elts_from_steps(ph.bsgs_required_steps(M), N))
    ctx = ph.context(p)
    ph.set_seed(4)
    sk = ph.secret_key(ctx).generate_sparse(ctx, 192)
    glk = sk.create_galois_keys(ctx)
    enc = ph.ckks_encoder(ctx)
    rng = np.random.default_rng(4)
    W = rng.uniform(-1 / 64, 1 / 64, (d_pad, d_pad))
    xv = rng.uniform(-1, 1, d_pad)
    scale = 2.0 ** 40
    t0 = time.perf_counter()
    diags = ph.pre_encode_bsgs_diagonals(ctx, enc, W.ravel(), d_pad, d_pad, d_pad, M, scale)
    t_encode = time.perf_counter() - t0
    x = sk.encrypt_symmetric(ctx, enc.encode_double_vector(ctx, np.tile(xv, enc.slot_count() // d_pad), scale))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    diags.expanded(ctx, x.chain_index())
    torch.cuda.synchronize()
    t_expand = time.perf_counter() - t0
    for _ in range(warmup):
        y = ph.bsgs_matmul_preencoded(ctx, glk, x, diags)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        y = ph.bsgs_matmul_preencoded(ctx, glk, x, diags)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    got = np.array(enc.decode_double_vector(ctx, sk.decrypt(ctx, y)))
    err = float(np.max(np.abs(got - np.tile(W @ xv, enc.slot_count() // d_pad))))
    # the tiled plaintext set the accumulation reads dominates the compulsory
    # bytes (5 bytes per residue on the 40-bit limbs, 8 on the 60-bit one)
    pt_bytes = ctx.native.bsgs_tiled_size(1, d_pad)
    del diags
    return {"ms": round(ms, 3), "max_abs_err": err, "encode_s": round(t_encode, 2),
            "expand_ms": round(t_expand * 1e3, 1), "plaintext_bytes": pt_bytes,
            "rotations": 2 * (M - 1), "chain": "{60, 40 x 19, 60 x 4}", "d_pad": d_pad, "baby": M,
            "giant": d_pad // M,
            "plaintexts": "the 4096 diagonals are expanded (residues + forward NTT) once per level and kept in "
                          "HBM (expand_ms, one-time, not in ms); the reference expands and transforms them inside "
                          "every product (src/bsgs.cu:270-312), so ms + expand_ms is its per-call workload"}


def time_bootstrap(torch, steps, warmup, evalmod="cheb63"):
    """benchmark config 5 through the pyPhantom API: N = 2^16, the 2^15 slots
    uniform in [-1, 1] (seeded), scale 2^40, sparse ternary secret h = 192
    with the ModRaise under an h = 192 encapsulation secret, |Q| = 30 and 6
    special primes (dnum = 5).  evalmod "cheb63": this build's pipeline on
    bootstrap_coeff_bits() (q0 60 | 13 x 40 | SlotToCoeff 3 x 50 | EvalMod
    10 x 60 | CoeffToSlot 3 x 60, special 60), the ciphertext entering at the
    bottom of the chain.  evalmod "k28_r3": the reference's pipeline
    (EvalRound with evalmod_k28_r3) on the reference engine's chain
    ckks_engine_coeff_bits() (q_msg 58 | 14 x 40 | 3 x 58 | 9 x 58 | 3 x 29,
    special 58), entering one level above the bottom, SlotToCoeff at user
    scale 2^40.  Times whole bootstraps with the keys and diagonals resident;
    reports the refreshed precision -log2(max |decrypted - input|)."""
    import math

    import numpy as np

    import pyPhantom as ph

    ref = evalmod == "k28_r3"
    bits = ph.ckks_engine_coeff_bits() if ref else ph.bootstrap_coeff_bits()
    p = ph.params(ph.scheme_type.ckks)
    p.set_poly_modulus_degree(N)
    p.set_coeff_modulus(ph.create_coeff_modulus(N, bits))
    p.set_special_modulus_size(6)
    p.set_galois_elts(ph.bootstrap_required_galois_elts(16))
    ctx = ph.context(p)
    ph.set_seed(5)
    sk = ph.secret_key(ctx).generate_sparse(ctx, 192)
    enc = ph.ckks_encoder(ctx)
    scale = 2.0 ** 40
    t0 = time.perf_counter()
    if ref:
        bk = ph.create_bootstrap_key(ctx, enc, sk, sparse_hamming_weight=192, eval_mod_levels=9, user_scale=scale)
    else:
        bk = ph.create_bootstrap_key(ctx, enc, sk, sparse_hamming_weight=192, evalmod="cheb63")
    torch.cuda.synchronize()
    t_key = time.perf_counter() - t0
    rng = np.random.default_rng(5)
    z = rng.uniform(-1, 1, enc.slot_count())
    ct = sk.encrypt_symmetric(ctx, enc.encode_double_vector(ctx, z, scale, ctx.size_Q - (1 if ref else 0)))
    for _ in range(warmup):
        out = ph.bootstrap(ctx, enc, ct, bk, scale)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        out = ph.bootstrap(ctx, enc, ct, bk, scale)
    e1.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    ms = e0.elapsed_time(e1) / steps
    got = np.array(enc.decode_double_vector(ctx, sk.decrypt(ctx, out)))
    err = float(np.max(np.abs(got - z)))
    chain = ("q_msg 58 | 14 x 40 | 3 x 58 | 9 x 58 | 3 x 29 + 6 x 58 special" if ref
             else "q0 60 | 13 x 40 | 3 x 50 | 10 x 60 | 3 x 60 + 6 x 60 special")
    r = {"ms": round(ms, 2), "wall_ms": round(wall_ms, 2), "precision_bits": round(-math.log2(err), 2),
         "max_abs_err": err, "keygen_s": round(t_key, 1), "galois_keys": len(bk.glk.keys),
         "levels_left": ctx.size_Ql(out.chain_index()) - 1, "evalmod": evalmod,
         "evalmod_levels": bk.eval_mod_levels, "chain": chain, "secret_h": 192}
    del bk
    torch.cuda.empty_cache()
    return r


def measured_traffic():
    """HBM bytes per forward NTT from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE of both kernels, scaled by the plain-copy factor);
    None if that summary is absent."""
    path = os.path.join(ROOT, "profiles", "ntt_fwd_N65536_2x35_traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get("traffic_bytes_per_forward_ntt")
    except (OSError, ValueError):
        return None


def cpu_baseline(mods, seconds, threads=1):
    """Oracle forward NTT on `threads` host threads (OpenMP over limbs), repeated
    over the config-2 batch for ~`seconds`."""
    import numpy as np

    import py_oracle as O

    orc = O.Oracle(N, mods, 1)
    rng = np.random.default_rng(0)
    x = np.stack([rng.integers(0, q, size=(POLYS, N), dtype=np.uint64) for q in mods[:LIMBS]], axis=1)
    limbs, t0 = 0, time.perf_counter()
    while True:
        orc.ntt_fwd(x, threads=threads)
        limbs += POLYS * LIMBS
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {"value": round(limbs / el, 2), "unit": "limbs/s", "cores": threads, "kind": "port",
            "sample": f"{limbs // (POLYS * LIMBS)} forward NTTs of the 2x35-limb N=2^16 batch "
                      f"({limbs} limbs, {el:.1f} s) by oracle/ckks_oracle.c (radix-2 Cooley-Tukey with "
                      f"precomputed Shoup twiddle pairs), {threads} thread{'s' if threads > 1 else ''}",
            "cpu": cpu_model(), "build": O.build_info()}


def cpu_model():
    """The host CPU's model name (from /proc/cpuinfo), or the platform string."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or platform.machine()


def host_threads():
    """Host threads this process may use (its CPU affinity, at most 16: the GPU
    box's share of the host for one GPU)."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-hmult", action="store_true")
    ap.add_argument("--no-bsgs", action="store_true")
    ap.add_argument("--no-boot", action="store_true")
    ap.add_argument("--mode", choices=["full", "ntt", "ntt-sweep", "copy", "hmult", "hmult35", "bsgs", "bootstrap"],
                    default="full",
                    help="ntt: only the NTT timing (for rocprofv3 kernel traces); ntt-sweep: forward and inverse "
                         "NTT time for 56 to 96 limbs; copy: the hand-written streaming copy of the "
                         "same 35 MiB batches (the plain-copy calibration of FETCH_SIZE / WRITE_SIZE); hmult: only "
                         "config-3 HMult + relin + rescale; hmult35: only the L=35 variant; bsgs: only the "
                         "config-4 matrix-vector product; bootstrap: only the config-5 bootstrap")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for {args.gpus}); the hot path "
              "would shard by RNS limb or by independent ciphertexts, neither of which is built here",
              file=sys.stderr)
        sys.exit(2)

    import torch

    import pfa_native as P

    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(2)
    mods = P.create_coeff_modulus(N, [50] * LIMBS + [60])
    ctx = P.NativeContext(N, mods, 1)
    n_batches = 10  # 10 x 35 MiB > 256 MiB Infinity Cache
    batches = [uniform(torch, (POLYS, LIMBS, N), mods, dev, gen) for _ in range(n_batches)]
    if args.mode == "bsgs":
        del batches
        r = time_bsgs(torch, max(2, args.steps // 40), 1)
        log(f"bench: bsgs mode, config 4: {r}")
        return
    if args.mode == "bootstrap":
        del batches
        r = time_bootstrap(torch, max(2, args.steps // 40), 1)
        log(f"bench: bootstrap mode, config 5: {r}")
        r = time_bootstrap(torch, max(2, args.steps // 40), 1, "k28_r3")
        log(f"bench: bootstrap mode, config 5 EvalRound: {r}")
        return
    if args.mode == "ntt-sweep":
        del batches
        print(json.dumps({"ntt_limb_sweep": ntt_limb_sweep(torch, P, dev, gen, args.steps)}))
        return
    if args.mode == "hmult":
        del batches
        r = time_hmult(torch, P, dev, gen, 24, 4, args.steps, args.warmup)
        log(f"bench: hmult mode, config 3: {r}")
        return
    if args.mode == "hmult35":
        del batches
        r = time_hmult(torch, P, dev, gen, 35, 1, args.steps, args.warmup)
        log(f"bench: hmult35 mode, L=35: {r}")
        return
    if args.mode == "copy":
        us = time_copy(torch, P, batches, args.steps, args.warmup)
        log(f"bench: {args.steps} streaming copies of {POLYS * LIMBS * LIMB_BYTES} bytes, {us:.2f} us each "
            f"({NTT_BYTES / (us * 1e-6) / 1e9:.0f} GB/s)")
        return
    log(f"bench: config 2 forward NTT, {args.steps} steps, {args.warmup} warmup, {n_batches} rotating batches")
    wall, ev_ms = time_ntt(torch, ctx, batches, args.steps, args.warmup)
    log(f"bench: forward done, {ev_ms * 1e3:.1f} us/launch")
    _, ev_inv_ms = time_ntt(torch, ctx, batches, args.steps, args.warmup, inverse=True)
    log(f"bench: inverse done, {ev_inv_ms * 1e3:.1f} us/launch")
    copy_us = time_copy(torch, P, batches, args.steps, args.warmup)
    log(f"bench: streaming copy of the batch {copy_us:.1f} us")
    limbs = POLYS * LIMBS
    # value, ms_per_step and the roofline all come from the same HIP-event
    # timing on the launch stream; the wall clock is reported beside them
    value = limbs / (ev_ms * 1e-3)
    achieved = NTT_BYTES / (ev_ms * 1e-3) / 1e9
    del batches
    torch.cuda.empty_cache()
    if args.mode == "ntt":
        log(f"bench: ntt mode done, forward {value:.1f} limbs/s")
        return

    hm = {}
    if not args.no_hmult:
        hm["config3_Q24_alpha4"] = time_hmult(torch, P, dev, gen, 24, 4, max(10, args.steps // 4), 5)
        log(f"bench: hmult config3 {hm['config3_Q24_alpha4']['ms']} ms")
        torch.cuda.empty_cache()
        hm["L35_Q35_alpha1"] = time_hmult(torch, P, dev, gen, 35, 1, max(5, args.steps // 10), 3)
        log(f"bench: hmult L=35 {hm['L35_Q35_alpha1']['ms']} ms")
        torch.cuda.empty_cache()

    bsgs = None
    if not args.no_bsgs:
        bsgs = time_bsgs(torch, 5, 1)
        log(f"bench: bsgs config4 {bsgs['ms']} ms, max abs err {bsgs['max_abs_err']:.2e}")
        torch.cuda.empty_cache()

    boot = boot_ref = None
    if not args.no_boot:
        boot = time_bootstrap(torch, 3, 1)
        log(f"bench: bootstrap config5 {boot['ms']} ms, {boot['precision_bits']} bits")
        boot_ref = time_bootstrap(torch, 3, 1, "k28_r3")
        log(f"bench: bootstrap config5 EvalRound {boot_ref['ms']} ms, {boot_ref['precision_bits']} bits")
        torch.cuda.empty_cache()

    cpu = cpu_all = None
    if not args.no_cpu:
        cpu = cpu_baseline(mods, args.cpu_seconds)
        log(f"bench: cpu baseline {cpu['value']} limbs/s")
        nt = host_threads()
        if nt > 1:
            cpu_all = cpu_baseline(mods, args.cpu_seconds / 2, nt)
            log(f"bench: cpu baseline on {nt} threads {cpu_all['value']} limbs/s")

    line = {
        "metric": "NTT limbs/s at N=2^16; HMult+relin+rescale ms (L=35); % HBM roofline",
        "value": round(value, 1),
        "unit": "limbs/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ev_ms, 5),
        "wall_ms_per_step": round(wall / args.steps * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u64",
        "data": "synthetic: uint64 residues uniform in [0, q_l) from a seeded torch generator",
        "config": {"workload": "config 2: batched forward NTT, N=2^16, 2 polys x 35 limbs (50-bit primes)",
                   "N": N, "polys": POLYS, "limbs": LIMBS, "rotating_batches": n_batches},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "traffic_source": "profiles/ntt_fwd_N65536_2x35_traffic.json: rocprofv3 --pmc FETCH_SIZE "
                                       "and WRITE_SIZE of both kernels, scaled by the plain-copy factors",
                     "kernel": "forward NTT (ntt_fwd_cols + ntt_fwd_rows), 16 B/residue algorithmic"},
        "cpu_baseline": cpu,
        "cpu_baseline_all_threads": cpu_all,
        "ntt_inverse_limbs_per_s": round(limbs / (ev_inv_ms * 1e-3), 1),
        "ntt_forward_us": round(ev_ms * 1e3, 2),
        "copy_ceiling": {"us": round(copy_us, 2), "GB_per_s": round(NTT_BYTES / (copy_us * 1e-6) / 1e9, 1),
                         "what": "pfa_stream_copy of the same 2x35-limb batch (73.4 MB moved), the achievable "
                                 "one-read-one-write time of a forward NTT"},
        "ntt_inverse_us": round(ev_inv_ms * 1e3, 2),
        "ntt_over_copy": round(ev_ms * 1e3 / copy_us, 3),
        "hmult_relin_rescale": hm,
        "bsgs_matvec_config4": bsgs,
        "bootstrap_config5": boot,
        "bootstrap_config5_evalround": boot_ref,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
