"""pyPhantom -- the reference's Python API (python/src/binding.cu) for the CKKS
hot path, running on the MI355X core through the C ABI (pfa_native).

Names, argument order and return conventions follow the pybind11 module
`pyPhantom` (binding.cu:23-290): `params`, `context`, `secret_key`,
`public_key`, `relin_key`, `galois_key`, `ckks_encoder`, `plaintext`,
`ciphertext`, and the evaluator functions (`add`, `sub`, `negate`,
`multiply`, `multiply_and_relin`, `relinearize`, `rescale_to_next`,
`mod_switch_*`, `multiply_plain`, `add_plain`, `apply_galois`, `rotate`,
`hoisting`, `hoist_rotations`, ...).  Operations return new objects, as the
reference's by-value bindings do (include/evaluate.cuh:134-139).  Errors are
ValueError for invalid arguments and RuntimeError otherwise, as pybind11 maps
the reference's std::invalid_argument / std::logic_error.

Every residue computation runs in libphantom_amd.so on the GPU.  Randomness
(secret, uniform masks, errors) is sampled on the host from numpy's seedable
generator and uploaded; the reference samples on the GPU with salsa20
(src/prng.cu), whose streams are not reproducible anyway (seeds come from
std::random_device).  Errors follow the reference's centred binomial
distribution with 21 + 21 coin flips (sigma ~ 3.24, src/prng.cu:222-243).
"""
from __future__ import annotations

import enum
import itertools
import struct
import threading

import numpy as np

import pfa_native as _N

__version__ = "amd-1"

_seed_counter = itertools.count()
_global_seed = None


def set_seed(seed: int | None) -> None:
    """Seed the host-side samplers (keys, masks, errors); None = OS entropy."""
    global _global_seed, _seed_counter
    _global_seed = seed
    _seed_counter = itertools.count()


def _rng(seed=None):
    if seed is not None:
        return np.random.default_rng(seed)
    if _global_seed is not None:
        return np.random.default_rng((_global_seed, next(_seed_counter)))
    return np.random.default_rng()


def _torch():
    import torch

    return torch


class scheme_type(enum.IntEnum):
    none = 0
    bfv = 1
    ckks = 2
    bgv = 3


class mul_tech_type(enum.IntEnum):
    none = 0
    behz = 1
    hps = 2
    hps_overq = 3
    hps_overq_leveled = 4


class sec_level_type(enum.IntEnum):
    """include/host/modulus.h security levels (binding.cu:46-50)."""
    none = 0
    tc128 = 128
    tc192 = 192
    tc256 = 256


class modulus(int):
    """arith::Modulus (include/host/modulus.h:14-80, binding.cu:53-54): a prime or
    zero of at most 61 bits.  An int subclass, so a list of them goes anywhere a
    list of moduli goes; `.value` is the reference's value()."""

    def __new__(cls, value: int = 0):
        v = int(value)
        # src/host/modulus.cu:15-24: 0 is allowed, 1 and values past 61 bits are not
        if v < 0 or v >> 61 or v == 1:
            raise ValueError("value can be at most 61-bit and cannot be 1")
        return super().__new__(cls, v)

    @property
    def value(self) -> int:
        return int(self)

    def bit_count(self) -> int:
        return int(self).bit_length()

    def is_zero(self) -> bool:
        return int(self) == 0

    def __repr__(self):
        return f"modulus({int(self)})"


def create_coeff_modulus(poly_modulus_degree: int, bit_sizes) -> list[modulus]:
    """CoeffModulus::Create (binding.cu:56): distinct NTT-friendly primes
    (p = 1 mod 2N) of the given bit sizes, in the reference's order."""
    return [modulus(p) for p in _N.create_coeff_modulus(poly_modulus_degree, list(bit_sizes))]


def create_plain_modulus(poly_modulus_degree: int, bit_size: int) -> modulus:
    """PlainModulus::Batching (binding.cu:58): one batching-friendly prime of the
    given size.  Only BFV/BGV parameters take it; `params.set_plain_modulus` of
    this CKKS core rejects it."""
    return create_coeff_modulus(poly_modulus_degree, [bit_size])[0]


class cuda_stream:
    """util::cuda_stream_wrapper (binding.cu:69-70): a new device stream at the
    default priority.  Used as a context manager, every call inside it runs on
    this stream, because this module launches on the calling thread's current
    stream."""

    def __init__(self):
        t = _torch()
        if not t.cuda.is_available():
            raise RuntimeError("cuda_stream: no GPU device is visible")
        self.stream = t.cuda.Stream()
        self._ctx = None

    def synchronize(self):
        self.stream.synchronize()

    def __enter__(self):
        self._ctx = _torch().cuda.stream(self.stream)
        self._ctx.__enter__()
        return self

    def __exit__(self, *exc):
        ctx, self._ctx = self._ctx, None
        return ctx.__exit__(*exc)


def set_cuda_device(device_id: int) -> None:
    """set_cuda_device (python/src/binding.cu:387-395): make device_id current for
    the calling thread (contexts and tensors created afterwards default to it)."""
    t = _torch()
    if not 0 <= int(device_id) < t.cuda.device_count():
        raise RuntimeError(f"set_cuda_device failed: no device {device_id}")
    t.cuda.set_device(int(device_id))


def get_cuda_device_count() -> int:
    """get_cuda_device_count (python/src/binding.cu:397-402): visible devices, 0 on error."""
    try:
        return int(_torch().cuda.device_count())
    except Exception:
        return 0


def get_elt_from_step(step: int, coeff_count: int) -> int:
    """include/galois.cuh:16-49."""
    return _N.galois_elt_from_step(step, coeff_count)


def get_elts_from_steps(steps, coeff_count: int) -> list[int]:
    return [get_elt_from_step(s, coeff_count) for s in steps]


class params:
    """EncryptionParameters (include/host/encryptionparams.h); CKKS only."""

    def __init__(self, scheme=scheme_type.ckks):
        if scheme != scheme_type.ckks:
            raise ValueError("this core implements the CKKS scheme only")
        self.scheme = scheme
        self.poly_modulus_degree = 0
        self.coeff_modulus = []
        self.special_modulus_size = 1
        self.galois_elts = []
        self.mul_tech = mul_tech_type.none

    def set_mul_tech(self, t):
        self.mul_tech = t

    def set_poly_modulus_degree(self, n):
        self.poly_modulus_degree = int(n)

    def set_special_modulus_size(self, k):
        self.special_modulus_size = int(k)

    def set_galois_elts(self, elts):
        self.galois_elts = [int(e) for e in elts]

    def set_coeff_modulus(self, mods):
        self.coeff_modulus = [int(getattr(m, "value", m)) for m in mods]

    def set_plain_modulus(self, _):
        raise ValueError("plain modulus is a BFV/BGV parameter")


class context:
    """PhantomContext (src/context.cu:121-183): chain index 0 = key level,
    chain c >= 1 holds |Q| - c + 1 data primes."""

    def __init__(self, parms: params, device: int | None = None):
        if not parms.poly_modulus_degree or not parms.coeff_modulus:
            raise ValueError("poly modulus degree and coefficient modulus must be set")
        self.parms = parms
        self.N = parms.poly_modulus_degree
        self.moduli = list(parms.coeff_modulus)
        self.size_P = parms.special_modulus_size
        self.size_Q = len(self.moduli) - self.size_P
        # the calling thread's current device unless given (set_cuda_device)
        self.device = _torch().cuda.current_device() if device is None else int(device)
        self.native = _N.NativeContext(self.N, self.moduli, self.size_P, self.device)
        self.galois_elts = list(parms.galois_elts)
        # device constants made on first use (monomials, constant plaintexts):
        # each upload would otherwise be one more host-to-device copy per call
        self._const_cache = {}
        self._const_lock = threading.Lock()

    def _cached_const(self, key, make):
        """The device constant `key`, made by make() once per context on the
        calling thread's current stream.  An event recorded after it is made
        orders every later use: a stream that first reads it waits for that
        event once (a device-side wait, the host does not block)."""
        t = _torch()
        stream = t.cuda.current_stream(self.device)
        with self._const_lock:
            hit = self._const_cache.get(key)
            if hit is None:
                data = make()
                ev = t.cuda.Event()
                ev.record(stream)
                hit = (data, ev, {stream.cuda_stream})
                self._const_cache[key] = hit
            data, ev, ready = hit
            if stream.cuda_stream not in ready:
                stream.wait_event(ev)
                ready.add(stream.cuda_stream)
        return data

    def total_parm_size(self) -> int:
        return self.size_Q + 1

    def get_first_index(self) -> int:
        return 1

    def size_Ql(self, chain_index: int) -> int:
        return self.size_Q - (chain_index - 1)

    @property
    def dnum(self) -> int:
        return self.size_Q // self.size_P

    @property
    def dev(self):
        return _torch().device("cuda", self.device)

    # ---- helpers (device tensors) ----
    def _empty(self, *shape):
        t = _torch()
        return t.empty(shape, dtype=t.uint64, device=self.dev)

    def _upload(self, a: np.ndarray):
        return _to_dev(np.ascontiguousarray(a, dtype=np.uint64), self.dev)

    def _signed_to_rns(self, coeffs: np.ndarray, L: int, start: int = 0):
        """Signed integer coefficients [N] -> residues [L][N] (coefficient form)."""
        c = _to_dev(np.ascontiguousarray(coeffs, dtype=np.int64), self.dev)
        out = self._empty(L, self.N)
        self.native.poly_from_signed(c, out, L, start)
        return out

    def _uniform(self, rng, L: int, start: int = 0):
        a = np.stack([rng.integers(0, q, size=self.N, dtype=np.uint64) for q in self.moduli[start:start + L]])
        return self._upload(a)

    def _cbd(self, rng):
        """Centred binomial error, 21 + 21 coins (src/prng.cu:222-243)."""
        return (rng.binomial(21, 0.5, self.N) - rng.binomial(21, 0.5, self.N)).astype(np.int64)

    def _ntt(self, t, L, start=0):
        self.native.ntt_forward(t, 1, L, start)
        return t


# ---------------------------------------------------------------- binary format
# The reference's save/load layout (include/ciphertext.h:173-214,
# include/plaintext.h:73-101, include/secretkey.h:99-111, :192-228, :290-318,
# :537-575): raw little-endian fields, no padding, then the residues as
# uint64 limbs in [poly][limb][N] order.
_CT_HEADER = struct.Struct("<QQQQdQQ??")  # chain_index, size, N, |Ql|, scale, correction_factor,
#                                           noiseScaleDeg, is_ntt_form, is_asymmetric
_PT_HEADER = struct.Struct("<QQQd")  # chain_index, N, |Ql|, scale
_SK_HEADER = struct.Struct("<QQQ")  # sk_max_power, N, |QP|
_COUNT = struct.Struct("<Q")  # dnum of a relin key, key count of a Galois key


def _read_exact(stream, n: int) -> bytes:
    b = stream.read(n)
    if len(b) != n:
        raise ValueError("unexpected end of stream")
    return b


def _write_limbs(stream, tensor):
    stream.write(np.ascontiguousarray(tensor.cpu().numpy(), dtype=np.uint64).tobytes())


def _to_dev(a: np.ndarray, dev):
    """Host array -> device tensor through pinned memory, queued on the current
    stream: a copy from pageable memory would make the host wait for all the
    work already queued, leaving the GPU idle while the next calls are issued."""
    t = _torch()
    return t.from_numpy(a).pin_memory().to(dev, non_blocking=True)


def _read_limbs(stream, shape, dev):
    n = int(np.prod(shape))
    a = np.frombuffer(_read_exact(stream, 8 * n), dtype=np.uint64).reshape(shape)
    return _torch().from_numpy(a.copy()).to(dev)


def _device(ctx):
    t = _torch()
    return ctx.dev if ctx is not None else t.device("cuda", t.cuda.current_device())


def _opened(stream, mode):
    """A path opens a file; a file object is used as given."""
    if isinstance(stream, (str, bytes)) or hasattr(stream, "__fspath__"):
        return open(stream, mode), True
    return stream, False


def _save_ct_record(stream, data, chain, scale, is_ntt=True, correction_factor=1, noise_scale_deg=1,
                    is_asymmetric=False):
    size, L, N = (int(x) for x in data.shape)
    stream.write(_CT_HEADER.pack(chain, size, N, L, float(scale), correction_factor, noise_scale_deg, bool(is_ntt),
                                 bool(is_asymmetric)))
    _write_limbs(stream, data)


def _load_ct_record(stream, dev):
    chain, size, N, L, scale, cf, nsd, ntt, asym = _CT_HEADER.unpack(_read_exact(stream, _CT_HEADER.size))
    if size < 1 or L < 1 or N < 2 or N & (N - 1) or size * L * N > (1 << 36):
        raise ValueError("corrupt ciphertext header")
    return _read_limbs(stream, (size, L, N), dev), chain, scale, cf, nsd, ntt, asym


class plaintext:
    def __init__(self):
        self.data = None
        self._chain_index = 0
        self._scale = 1.0

    def chain_index(self) -> int:
        return self._chain_index

    def scale(self) -> float:
        return self._scale

    def save(self, stream):
        """PhantomPlaintext::save (include/plaintext.h:73-85)."""
        f, own = _opened(stream, "wb")
        try:
            L, N = (int(x) for x in self.data.shape)
            f.write(_PT_HEADER.pack(self._chain_index, N, L, float(self._scale)))
            _write_limbs(f, self.data)
        finally:
            if own:
                f.close()

    def load(self, stream, ctx: context | None = None):
        """PhantomPlaintext::load (include/plaintext.h:87-101)."""
        f, own = _opened(stream, "rb")
        try:
            chain, N, L, scale = _PT_HEADER.unpack(_read_exact(f, _PT_HEADER.size))
            self.data = _read_limbs(f, (L, N), _device(ctx))
            self._chain_index, self._scale = chain, scale
        finally:
            if own:
                f.close()
        return self


class ciphertext:
    """PhantomCiphertext (include/ciphertext.h): data [size][|Ql|][N] in NTT form."""

    def __init__(self):
        self.data = None
        self._chain_index = 0
        self._scale = 1.0
        self.is_ntt_form = True
        # > 1: a bundle of that many size-2 ciphertexts at one level and scale,
        # data [2 members][|Ql|][N], that the evaluator steps in lockstep with
        # batched native calls (bootstrap's EvalMod tracks)
        self._members = 1

    def chain_index(self) -> int:
        return self._chain_index

    def scale(self) -> float:
        return self._scale

    def set_scale(self, s: float):
        self._scale = float(s)

    def size(self) -> int:
        return 0 if self.data is None else int(self.data.shape[0])

    def _like(self, data, chain=None, scale=None):
        c = ciphertext()
        c.data = data
        c._chain_index = self._chain_index if chain is None else chain
        c._scale = self._scale if scale is None else scale
        c._members = self._members
        return c

    def save(self, stream):
        """PhantomCiphertext::save (include/ciphertext.h:173-191)."""
        f, own = _opened(stream, "wb")
        try:
            _save_ct_record(f, self.data, self._chain_index, self._scale, self.is_ntt_form,
                            getattr(self, "correction_factor", 1), getattr(self, "noise_scale_deg", 1),
                            getattr(self, "is_asymmetric", False))
        finally:
            if own:
                f.close()

    def load(self, stream, ctx: context | None = None):
        """PhantomCiphertext::load (include/ciphertext.h:193-214); ctx picks the device."""
        f, own = _opened(stream, "rb")
        try:
            (self.data, self._chain_index, self._scale, self.correction_factor, self.noise_scale_deg,
             self.is_ntt_form, self.is_asymmetric) = _load_ct_record(f, _device(ctx))
        finally:
            if own:
                f.close()
        return self


class _ksk:
    """Key switching key material: [dnum][2][|QP|][N] on the device."""

    def __init__(self, data):
        self.data = data


def _save_ksk(stream, data):
    """PhantomRelinKey::save (include/secretkey.h:192-204): dnum, then each
    digit as a key-level ciphertext [2][|QP|][N]."""
    if data is None:
        raise ValueError("key has not been generated")
    stream.write(_COUNT.pack(int(data.shape[0])))
    for d in range(int(data.shape[0])):
        _save_ct_record(stream, data[d], 0, 1.0)


def _load_ksk(stream, dev):
    (dnum,) = _COUNT.unpack(_read_exact(stream, _COUNT.size))
    digits = [_load_ct_record(stream, dev)[0] for _ in range(dnum)]
    if not digits:
        raise ValueError("key has no digits")
    return _torch().stack(digits).contiguous()


class relin_key(_ksk):
    def __init__(self, data=None):
        super().__init__(data)

    def save(self, stream):
        f, own = _opened(stream, "wb")
        try:
            _save_ksk(f, self.data)
        finally:
            if own:
                f.close()

    def load(self, stream, ctx: context | None = None):
        """PhantomRelinKey::load (include/secretkey.h:206-228)."""
        f, own = _opened(stream, "rb")
        try:
            self.data = _load_ksk(f, _device(ctx))
        finally:
            if own:
                f.close()
        return self


class galois_key:
    def __init__(self, elts=None):
        self.keys = {}  # Galois element -> key tensor
        # the context's galois_elts: the reference keeps one key slot per
        # element in this order (PhantomGaloisKey::relin_keys_)
        self.elts = list(elts) if elts is not None else None

    def get(self, elt):
        k = self.keys.get(elt)
        if k is None:
            raise RuntimeError(f"Galois key not present for element {elt}")
        return k

    def save(self, stream):
        """PhantomGaloisKey::save (include/secretkey.h:290-302): the key count,
        then one relin-key record per Galois element in the context's order.
        As in the reference, an element without a generated key (a set made by
        create_galois_keys_per_level for some elements only) is an error."""
        if not self.keys:
            raise ValueError("PhantomGaloisKey has not been generated")
        elts = self.elts if self.elts is not None else list(self.keys)
        missing = [e for e in elts if e not in self.keys]
        if missing:
            raise ValueError(f"PhantomRelinKey has not been generated (no key for Galois element {missing[0]})")
        f, own = _opened(stream, "wb")
        try:
            f.write(_COUNT.pack(len(elts)))
            for e in elts:
                _save_ksk(f, self.keys[e])
        finally:
            if own:
                f.close()

    def load(self, stream, ctx: context):
        """PhantomGaloisKey::load (include/secretkey.h:304-318); the elements
        come from ctx.galois_elts, as the file holds only the keys."""
        f, own = _opened(stream, "rb")
        try:
            (n,) = _COUNT.unpack(_read_exact(f, _COUNT.size))
            if n != len(ctx.galois_elts):
                raise ValueError(f"file holds {n} Galois keys, the context has {len(ctx.galois_elts)} elements")
            self.keys = {e: _load_ksk(f, ctx.dev) for e in ctx.galois_elts}
            self.elts = list(ctx.galois_elts)
        finally:
            if own:
                f.close()
        return self


class public_key:
    """PhantomPublicKey: (-(a s + e), a) over every prime of the key level, NTT form."""

    def __init__(self, ctx: context | None = None, data=None):
        self.ctx = ctx
        self.data = data

    def save(self, stream):
        """PhantomPublicKey::save (include/secretkey.h:99-104): one ciphertext record."""
        if self.data is None:
            raise ValueError("PhantomPublicKey has not been generated")
        f, own = _opened(stream, "wb")
        try:
            _save_ct_record(f, self.data, 0, 1.0)
        finally:
            if own:
                f.close()

    def load(self, stream, ctx: context | None = None):
        f, own = _opened(stream, "rb")
        try:
            self.data = _load_ct_record(f, _device(ctx))[0]
            self.ctx = ctx
        finally:
            if own:
                f.close()
        return self

    def encrypt_asymmetric(self, ctx: context, pt: plaintext, seed=None) -> ciphertext:
        """ct = (pk0 u + e0 + m, pk1 u + e1) over the plaintext's primes."""
        if self.data is None:
            raise ValueError("public key is empty")
        rng = _rng(seed)
        L = ctx.size_Ql(pt.chain_index())
        nat = ctx.native
        u = ctx._ntt(ctx._signed_to_rns(rng.integers(-1, 2, ctx.N), L), L)
        out = ctx._empty(2, L, ctx.N)
        for k in range(2):
            e = ctx._ntt(ctx._signed_to_rns(ctx._cbd(rng), L), L)
            nat.poly_mul(self.data[k, :L].contiguous(), u, out[k], L)
            nat.poly_add(out[k], e, out[k], L)
        nat.poly_add(out[0], pt.data, out[0], L)
        ct = ciphertext()
        ct.data, ct._chain_index, ct._scale = out, pt.chain_index(), pt.scale()
        return ct


class secret_key:
    """PhantomSecretKey (src/secretkey.cu): ternary secret, NTT form over all |QP| primes."""

    def __init__(self, ctx: context | None = None, seed=None):
        self.sk = None
        self.coeffs = None
        if ctx is not None:
            rng = _rng(seed)
            self._set(ctx, rng.integers(-1, 2, ctx.N).astype(np.int64))

    def _set(self, ctx, coeffs):
        self.ctx = ctx
        self.coeffs = coeffs
        QP = len(ctx.moduli)
        self.sk = ctx._ntt(ctx._signed_to_rns(coeffs, QP), QP)

    def generate_sparse(self, ctx: context, hamming_weight: int, seed=None):
        """Sparse ternary secret with `hamming_weight` nonzeros (src/secretkey.cu:513-576)."""
        if not 0 < hamming_weight <= ctx.N:
            raise ValueError("hamming weight out of range")
        rng = _rng(seed)
        c = np.zeros(ctx.N, dtype=np.int64)
        idx = rng.choice(ctx.N, size=hamming_weight, replace=False)
        c[idx] = rng.choice(np.array([-1, 1], dtype=np.int64), size=hamming_weight)
        self._set(ctx, c)
        return self

    def _require(self):
        if self.sk is None:
            raise ValueError("secret key is not generated")

    def save(self, stream):
        """PhantomSecretKey::save (include/secretkey.h:537-554): sk_max_power
        (1 for CKKS), N, |QP|, then s in NTT form over every prime."""
        self._require()
        f, own = _opened(stream, "wb")
        try:
            QP, N = (int(x) for x in self.sk.shape)
            f.write(_SK_HEADER.pack(1, N, QP))
            _write_limbs(f, self.sk)
        finally:
            if own:
                f.close()

    def load(self, stream, ctx: context):
        """PhantomSecretKey::load (include/secretkey.h:556-575); only the first
        power is kept (CKKS uses s alone)."""
        f, own = _opened(stream, "rb")
        try:
            power, N, QP = _SK_HEADER.unpack(_read_exact(f, _SK_HEADER.size))
            if N != ctx.N or QP != len(ctx.moduli) or power < 1:
                raise ValueError("secret key does not match the context")
            data = _read_limbs(f, (power, QP, N), ctx.dev)
            self.ctx, self.sk, self.coeffs = ctx, data[0].contiguous(), None
        finally:
            if own:
                f.close()
        return self

    def _kswitch_key(self, ctx, new_key, rng):
        """generate_one_kswitch_key (src/secretkey.cu:354-398) via pfa_kswitch_key."""
        QP = len(ctx.moduli)
        dnum = ctx.dnum
        a = _torch().stack([ctx._uniform(rng, QP) for _ in range(dnum)])
        e = _torch().stack([ctx._ntt(ctx._signed_to_rns(ctx._cbd(rng), QP), QP) for _ in range(dnum)])
        out = ctx._empty(dnum, 2, QP, ctx.N)
        ctx.native.kswitch_key(new_key, self.sk, a.contiguous(), e.contiguous(), out)
        return out

    def gen_publickey(self, ctx: context, seed=None) -> public_key:
        """(-(a s + e), a) at the key level, over every prime (src/secretkey.cu:578-590)."""
        self._require()
        rng = _rng(seed)
        QP = len(ctx.moduli)
        a = ctx._uniform(rng, QP)
        e = ctx._ntt(ctx._signed_to_rns(ctx._cbd(rng), QP), QP)
        pk = ctx._empty(2, QP, ctx.N)
        nat = ctx.native
        nat.poly_mul(a, self.sk, pk[0], QP)
        nat.poly_add(pk[0], e, pk[0], QP)
        nat.poly_negate(pk[0], pk[0], QP)
        pk[1].copy_(a)
        return public_key(ctx, pk)

    def gen_relinkey(self, ctx: context, seed=None) -> relin_key:
        """Key for s^2 (src/secretkey.cu:592-615)."""
        self._require()
        QP = len(ctx.moduli)
        s2 = ctx._empty(QP, ctx.N)
        ctx.native.poly_mul(self.sk, self.sk, s2, QP)
        return relin_key(self._kswitch_key(ctx, s2, _rng(seed)))

    def _galois_key_for(self, ctx, elt, rng, digits=None):
        """Key for sigma_elt(s); with `digits`, only that many leading partitions
        (generate_one_kswitch_key_at_level, src/secretkey.cu:400-472: the same
        structure over every prime, the partitions a level does not use left out)."""
        QP = len(ctx.moduli)
        rot = ctx._empty(QP, ctx.N)
        ctx.native.apply_galois_ntt(elt, self.sk, rot, QP)
        key = self._kswitch_key(ctx, rot, rng)
        return key if digits is None or digits == key.shape[0] else key[:digits].contiguous()

    @staticmethod
    def _level_digits(ctx, target_chain_index: int):
        """Partitions a key for target_chain_index needs (0: the key level, all
        of them): ceil(|Ql| / |P|), src/secretkey.cu:423-435."""
        if target_chain_index == 0:
            return None
        if not 1 <= target_chain_index <= ctx.size_Q:
            raise ValueError("generate_one_kswitch_key_at_level: target_chain_index out of range")
        beta = -(-ctx.size_Ql(target_chain_index) // ctx.size_P)
        if beta > ctx.dnum:
            raise RuntimeError("generate_one_kswitch_key_at_level: computed beta_k is invalid")
        return beta

    def _elt_at(self, ctx, idx: int, what: str) -> int:
        if not 0 <= idx < len(ctx.galois_elts):
            raise IndexError(f"{what}: index out of range")
        elt = ctx.galois_elts[idx]
        if not (elt & 1) or elt >= 2 * ctx.N:
            raise ValueError(f"{what}: Galois element is not valid")
        return elt

    def create_galois_keys(self, ctx: context, seed=None) -> galois_key:
        """Keys for every element in params.galois_elts (src/secretkey.cu:642-682)."""
        self._require()
        rng = _rng(seed)
        g = galois_key(ctx.galois_elts)
        for elt in ctx.galois_elts:
            g.keys[elt] = self._galois_key_for(ctx, elt, rng)
        return g

    def create_galois_keys_per_level(self, ctx: context, indices, target_chain_indices, seed=None) -> galois_key:
        """create_galois_keys_per_level (src/secretkey.cu:726-775): keys for the
        Galois elements at positions `indices` of params.galois_elts, each with
        the partitions its target chain index needs (0: all); the other
        elements get no key."""
        self._require()
        indices, targets = list(indices), list(target_chain_indices)
        if len(indices) != len(targets):
            raise ValueError("create_galois_keys_per_level: indices and target_chain_indices must have the same length")
        rng = _rng(seed)
        g = galois_key(ctx.galois_elts)
        for idx, tci in zip(indices, targets):
            elt = self._elt_at(ctx, idx, "create_galois_keys_per_level")
            g.keys[elt] = self._galois_key_for(ctx, elt, rng, self._level_digits(ctx, tci))
        return g

    def create_one_galois_key(self, ctx: context, galois_elt_idx: int, target_chain_index: int = 0, seed=None):
        """create_one_galois_key (src/secretkey.cu:777-811): the key of one
        element, with the partitions target_chain_index needs (0: all)."""
        self._require()
        elt = self._elt_at(ctx, galois_elt_idx, "create_one_galois_key")
        return relin_key(self._galois_key_for(ctx, elt, _rng(seed), self._level_digits(ctx, target_chain_index)))

    def encrypt_symmetric(self, ctx: context, pt: plaintext, seed=None) -> ciphertext:
        """ct = (-a s + e + m, a) over the plaintext's primes."""
        self._require()
        rng = _rng(seed)
        L = ctx.size_Ql(pt.chain_index())
        nat = ctx.native
        a = ctx._uniform(rng, L)
        e = ctx._ntt(ctx._signed_to_rns(ctx._cbd(rng), L), L)
        out = ctx._empty(2, L, ctx.N)
        nat.poly_mul(a, self.sk[:L].contiguous(), out[0], L)
        nat.poly_negate(out[0], out[0], L)
        nat.poly_add(out[0], e, out[0], L)
        nat.poly_add(out[0], pt.data, out[0], L)
        out[1].copy_(a)
        ct = ciphertext()
        ct.data, ct._chain_index, ct._scale = out, pt.chain_index(), pt.scale()
        return ct

    def decrypt(self, ctx: context, ct: ciphertext) -> plaintext:
        """m = c0 + c1 s (+ c2 s^2) over the ciphertext's primes."""
        self._require()
        L = ctx.size_Ql(ct.chain_index())
        nat = ctx.native
        s = self.sk[:L].contiguous()
        m = ct.data[0].clone()
        t = ctx._empty(L, ctx.N)
        sp = s.clone()
        for i in range(1, ct.size()):
            nat.poly_mul(ct.data[i], sp, t, L)
            nat.poly_add(m, t, m, L)
            if i + 1 < ct.size():
                nat.poly_mul(sp, s, sp, L)
        pt = plaintext()
        pt.data, pt._chain_index, pt._scale = m, ct.chain_index(), ct.scale()
        return pt


class ckks_encoder:
    """PhantomCKKSEncoder (src/ckks.cu): N/2 complex slots, rotation group 5^j."""

    def __init__(self, ctx: context):
        self.ctx = ctx
        self._slots = ctx.N // 2

    def slot_count(self) -> int:
        return self._slots

    def _encode(self, ctx, values, scale, chain_index):
        t = _torch()
        v = np.asarray(values, dtype=np.complex128).ravel()
        if v.size == 0:
            raise ValueError("Input vector is empty")
        if v.size > self._slots:
            raise ValueError("Input vector exceeds max slots")
        if not 1 <= chain_index <= ctx.size_Q:
            raise ValueError("chain index out of range")
        L = ctx.size_Ql(chain_index)
        out = ctx._empty(L, ctx.N)
        ctx.native.ckks_encode(t.from_numpy(v).to(ctx.dev), scale, out, L)
        pt = plaintext()
        pt.data, pt._chain_index, pt._scale = out, chain_index, float(scale)
        return pt

    def encode_double_vector(self, ctx, values, scale, chain_index=1):
        return self._encode(ctx, np.asarray(values, dtype=np.float64), scale, chain_index)

    def encode_complex_vector(self, ctx, values, scale, chain_index=1):
        return self._encode(ctx, values, scale, chain_index)

    def _decode(self, ctx, pt):
        t = _torch()
        out = t.empty(self._slots, dtype=t.complex128, device=ctx.dev)
        ctx.native.ckks_decode(pt.data, pt.data.shape[0], pt.scale(), out)
        t.cuda.synchronize(ctx.dev)
        return out.cpu().numpy()

    def decode_complex_vector(self, ctx, pt):
        return self._decode(ctx, pt).tolist()

    def decode_double_vector(self, ctx, pt):
        return self._decode(ctx, pt).real.tolist()


# ---------------------------------------------------------------- evaluator
def _check_same(a: ciphertext, b: ciphertext):
    if a.chain_index() != b.chain_index():
        raise ValueError("encrypted1 and encrypted2 parameter mismatch")


def _check_scale(a, b):
    if abs(a.scale() - b.scale()) > 1e-9 * max(abs(a.scale()), 1.0):
        raise ValueError("scale mismatch")


def _signed_sum(ctx: context, like: ciphertext, terms) -> ciphertext:
    """sum_t k_t x_t over every poly of ciphertexts shaped like `like`, as one
    pfa_ct_lincomb launch (weights +-1: canonical sums, the same residues as
    the polynomial-wise add / sub / negate of src/evaluate.cu)."""
    L = ctx.size_Ql(like.chain_index())
    out = ctx._empty(*like.data.shape)
    ctx.native.ct_lincomb(L, [x.data for x, _ in terms], [k for _, k in terms], out)
    return like._like(out)


def negate(ctx: context, ct: ciphertext) -> ciphertext:
    return _signed_sum(ctx, ct, [(ct, -1)])


def add(ctx: context, a: ciphertext, b: ciphertext) -> ciphertext:
    _check_same(a, b)
    _check_scale(a, b)
    if a.size() != b.size():
        raise ValueError("ciphertext sizes differ")
    return _signed_sum(ctx, a, [(a, 1), (b, 1)])


def add_many(ctx: context, cts, _unused=None) -> ciphertext:
    """add_many (src/evaluate.cu): up to 8 ciphertexts per launch."""
    if not cts:
        raise ValueError("empty list")
    for c in cts[1:]:
        _check_same(cts[0], c)
        _check_scale(cts[0], c)
        if c.size() != cts[0].size():
            raise ValueError("ciphertext sizes differ")
    acc, rest = cts[0], list(cts[1:])
    while rest:
        chunk, rest = rest[:7], rest[7:]
        acc = _signed_sum(ctx, acc, [(acc, 1)] + [(c, 1) for c in chunk])
    return acc


def sub(ctx: context, a: ciphertext, b: ciphertext, negate: bool = False) -> ciphertext:
    _check_same(a, b)
    _check_scale(a, b)
    if a.size() != b.size():
        raise ValueError("ciphertext sizes differ")
    return _signed_sum(ctx, a, [(a, -1), (b, 1)] if negate else [(a, 1), (b, -1)])


def add_plain(ctx: context, ct: ciphertext, pt: plaintext) -> ciphertext:
    if ct.chain_index() != pt.chain_index():
        raise ValueError("encrypted and plain parameter mismatch")
    _check_scale(ct, pt)
    L = ctx.size_Ql(ct.chain_index())
    out = ct.data.clone()
    ctx.native.poly_add(ct.data[0], pt.data, out[0], L)
    return ct._like(out)


def sub_plain(ctx: context, ct: ciphertext, pt: plaintext) -> ciphertext:
    if ct.chain_index() != pt.chain_index():
        raise ValueError("encrypted and plain parameter mismatch")
    _check_scale(ct, pt)
    L = ctx.size_Ql(ct.chain_index())
    out = ct.data.clone()
    ctx.native.poly_sub(ct.data[0], pt.data, out[0], L)
    return ct._like(out)


def multiply_plain(ctx: context, ct: ciphertext, pt: plaintext) -> ciphertext:
    if ct.chain_index() != pt.chain_index():
        raise ValueError("encrypted and plain parameter mismatch")
    L = ctx.size_Ql(ct.chain_index())
    out = ctx._empty(*ct.data.shape)
    ctx.native.ct_multiply_plain(ct.data, pt.data, out, L)
    return ct._like(out, scale=ct.scale() * pt.scale())


def multiply(ctx: context, a: ciphertext, b: ciphertext) -> ciphertext:
    """Tensor product of two size-2 ciphertexts -> size 3 (src/evaluate.cu:345-397)."""
    _check_same(a, b)
    if a.size() != 2 or b.size() != 2:
        raise ValueError("multiply expects size-2 ciphertexts")
    L = ctx.size_Ql(a.chain_index())
    out = ctx._empty(3, L, ctx.N)
    ctx.native.tensor(a.chain_index(), a.data, b.data, out)
    return a._like(out, scale=a.scale() * b.scale())


def relinearize(ctx: context, ct: ciphertext, rlk: relin_key) -> ciphertext:
    if ct.size() != 3:
        raise ValueError("relinearize expects a size-3 ciphertext")
    L = ctx.size_Ql(ct.chain_index())
    out = ctx._empty(2, L, ctx.N)
    ctx.native.relinearize(ct.chain_index(), ct.data, rlk.data, out)
    return ct._like(out)


def _bundle_pair(a: ciphertext, b: ciphertext) -> int:
    """Members of a (bundle) operand pair of a multiplication; checks shapes."""
    m = a._members
    if b._members != m or a.size() != 2 * m or b.size() != 2 * m:
        raise ValueError("multiply_and_relin expects size-2 ciphertexts")
    return m


def multiply_and_relin(ctx: context, a: ciphertext, b: ciphertext, rlk: relin_key) -> ciphertext:
    """src/evaluate.cu:1061-1104 (bundles: every member in one batched call,
    pfa_multiply_and_relin_batch)."""
    _check_same(a, b)
    m = _bundle_pair(a, b)
    L = ctx.size_Ql(a.chain_index())
    out = ctx._empty(2 * m, L, ctx.N)
    if m == 1:
        ctx.native.multiply_and_relin(a.chain_index(), a.data, b.data, rlk.data, out)
    else:
        ctx.native.multiply_and_relin_batch(a.chain_index(), m, a.data, b.data, rlk.data, out)
    return a._like(out, scale=a.scale() * b.scale())


def _ntt_check(ctx: context, inout, coeff_modulus_size: int, start_modulus_idx: int, batch: int):
    t = _torch()
    if not isinstance(inout, t.Tensor) or inout.dtype != t.uint64 or inout.device.type != "cuda":
        raise ValueError("ntt: inout must be a torch.uint64 tensor on the context's device")
    if not inout.is_contiguous():
        raise ValueError("ntt: inout must be contiguous")
    if batch < 1 or coeff_modulus_size < 1:
        raise ValueError("ntt: empty batch")
    if inout.numel() != batch * coeff_modulus_size * ctx.N:
        raise ValueError(f"ntt: inout holds {inout.numel()} residues, expected batch x coeff_modulus_size x N = "
                         f"{batch * coeff_modulus_size * ctx.N}")
    if start_modulus_idx < 0 or start_modulus_idx + coeff_modulus_size > len(ctx.moduli):
        raise ValueError("ntt: limb range exceeds the context's primes")


def ntt_forward(ctx: context, inout, coeff_modulus_size: int, start_modulus_idx: int = 0, batch: int = 1,
                stream=None) -> None:
    """nwt_2d_radix8_forward_inplace[_batched] (include/ntt.cuh:173, :184): in
    place, `batch` polys x coeff_modulus_size limbs (limb-major, N residues
    each, a contiguous torch.uint64 device tensor); limb l uses the table row of
    prime start_modulus_idx + l.  Output in the reference's bit-reversed NTT
    order.  stream: a hipStream_t handle (default torch's current stream).  The
    reference exposes no NTT to Python; this follows the C++ signature."""
    _ntt_check(ctx, inout, coeff_modulus_size, start_modulus_idx, batch)
    ctx.native.ntt_forward(inout, batch, coeff_modulus_size, start_modulus_idx, stream)


def ntt_inverse(ctx: context, inout, coeff_modulus_size: int, start_modulus_idx: int = 0, batch: int = 1,
                stream=None) -> None:
    """nwt_2d_radix8_backward_inplace (include/ntt.cuh:216), batched like
    ntt_forward: the exact inverse, canonical residues."""
    _ntt_check(ctx, inout, coeff_modulus_size, start_modulus_idx, batch)
    ctx.native.ntt_inverse(inout, batch, coeff_modulus_size, start_modulus_idx, stream)


def synchronize(ctx: context, stream=None) -> None:
    """Waits for the context's work on `stream` (default torch's current
    stream) and raises RuntimeError if a kernel recorded an error on the device
    (pfa_synchronize)."""
    ctx.native.synchronize(stream)


def rescale_to_next(ctx: context, ct: ciphertext) -> ciphertext:
    """Floor division by q_last (src/evaluate.cu:1582-1602, src/rns.cu:1128-1184)."""
    L = ctx.size_Ql(ct.chain_index())
    if L < 2:
        raise ValueError("end of modulus switching chain reached")
    out = ctx._empty(ct.size(), L - 1, ctx.N)
    ctx.native.rescale(ct.chain_index(), ct.data, out)
    return ct._like(out, chain=ct.chain_index() + 1, scale=ct.scale() / ctx.moduli[L - 1])


def multiply_and_relin_rescale(ctx: context, a: ciphertext, b: ciphertext, rlk: relin_key) -> ciphertext:
    """rescale_to_next(multiply_and_relin(a, b)) as one native call
    (pfa_multiply_relin_rescale), bit-identical to the two calls: the
    relinearized product at full level is never formed.  The reference has no
    single call for this pair (src/evaluate.cu:1061-1104 then :1582-1602)."""
    _check_same(a, b)
    m = _bundle_pair(a, b)
    L = ctx.size_Ql(a.chain_index())
    if L < 2:
        raise ValueError("end of modulus switching chain reached")
    out = ctx._empty(2 * m, L - 1, ctx.N)
    if m == 1:
        ctx.native.multiply_relin_rescale(a.chain_index(), a.data, b.data, rlk.data, out)
    else:
        ctx.native.multiply_relin_rescale_batch(a.chain_index(), m, a.data, b.data, rlk.data, out)
    return a._like(out, chain=a.chain_index() + 1, scale=a.scale() * b.scale() / ctx.moduli[L - 1])


def relinearize_rescale(ctx: context, ct: ciphertext, rlk: relin_key) -> ciphertext:
    """rescale_to_next(relinearize(ct)) as one native call (pfa_relinearize_rescale),
    bit-identical to the two calls."""
    if ct.size() != 3:
        raise ValueError("relinearize expects a size-3 ciphertext")
    L = ctx.size_Ql(ct.chain_index())
    if L < 2:
        raise ValueError("end of modulus switching chain reached")
    out = ctx._empty(2, L - 1, ctx.N)
    ctx.native.relinearize_rescale(ct.chain_index(), ct.data, rlk.data, out)
    return ct._like(out, chain=ct.chain_index() + 1, scale=ct.scale() / ctx.moduli[L - 1])


def mod_switch_to_next(ctx: context, obj):
    """CKKS modulus drop: remove the last prime, keep the scale."""
    chain = obj.chain_index()
    L = ctx.size_Ql(chain)
    if L < 2:
        raise ValueError("end of modulus switching chain reached")
    if isinstance(obj, plaintext):
        pt = plaintext()
        pt.data, pt._chain_index, pt._scale = obj.data[:L - 1].contiguous(), chain + 1, obj.scale()
        return pt
    return obj._like(_drop_limbs(ctx, obj.data, L - 1), chain=chain + 1)


def _drop_limbs(ctx: context, data, L: int):
    """The first L limbs of every poly of [size][L'][N] data, as one launch:
    a one-term weighted sum with weight 1 reads each poly's first L limbs at
    the input's own poly stride (canonical residues, copied unchanged)."""
    out = ctx._empty(data.shape[0], L, data.shape[2])
    ctx.native.ct_lincomb(L, [data], [1], out)
    return out


def mod_switch_to(ctx: context, obj, chain_index: int):
    """Drops the primes above chain_index's level in one copy (the same limbs
    as repeated mod_switch_to_next, which copies once per prime)."""
    if chain_index < obj.chain_index():
        raise ValueError("cannot switch to a higher level modulus")
    if chain_index == obj.chain_index():
        return obj
    if chain_index > ctx.size_Q:
        raise ValueError("end of modulus switching chain reached")
    L = ctx.size_Ql(chain_index)
    if isinstance(obj, plaintext):
        pt = plaintext()
        pt.data, pt._chain_index, pt._scale = obj.data[:L].contiguous(), chain_index, obj.scale()
        return pt
    return obj._like(_drop_limbs(ctx, obj.data, L), chain=chain_index)


def mod_switch_to_inplace(ctx: context, obj, chain_index: int) -> None:
    r = mod_switch_to(ctx, obj, chain_index)
    obj.data, obj._chain_index = r.data, r._chain_index


def _apply_galois_key(ctx: context, ct: ciphertext, elt: int, key) -> ciphertext:
    """apply_galois_with_ksk (src/evaluate.cu:1607-1656) into a new ciphertext:
    a rotation batch of one, which reads ct and writes the output (the same
    residues as the in-place pfa_apply_galois, without copying ct first)."""
    if ct.size() != 2:
        raise ValueError("ciphertext size must be 2")
    out = ctx._empty(*ct.data.shape)
    ctx.native.rotate_batch(ct.chain_index(), ct.data.contiguous(), [elt], [key], out)
    return ct._like(out)


def apply_galois(ctx: context, ct: ciphertext, elt: int, glk: galois_key) -> ciphertext:
    """apply_galois_with_ksk (src/evaluate.cu:1607-1656)."""
    return _apply_galois_key(ctx, ct, elt, glk.get(elt))


def apply_galois_with_key(ctx: context, ct: ciphertext, elt: int, key: relin_key) -> ciphertext:
    return _apply_galois_key(ctx, ct, elt, key.data)


def _naf(step: int):
    """Non-adjacent form digits (+-2^k) of step, least significant first, from
    |step| with the sign applied afterwards (include/host/numth.h:17-34)."""
    sign, v, out, i = step < 0, abs(step), [], 0
    while v:
        z = 2 - (v & 3) if v & 1 else 0
        v = (v - z) >> 1
        if z:
            out.append((-z if sign else z) * (1 << i))
        i += 1
    return out


def rotate(ctx: context, ct: ciphertext, step: int, glk: galois_key) -> ciphertext:
    """rotate_internal (src/evaluate.cu:1683-1713): direct key, else NAF decomposition."""
    elt = get_elt_from_step(step, ctx.N)
    if elt in glk.keys:
        return apply_galois(ctx, ct, elt, glk)
    digits = _naf(step)
    if len(digits) <= 1:
        raise ValueError("Galois key not present")
    out = ct
    for d in digits:
        if abs(d) != ctx.N // 2:
            out = rotate(ctx, out, d, glk)
    return out


def rotate_with_key(ctx: context, ct: ciphertext, step: int, key: relin_key) -> ciphertext:
    return apply_galois_with_key(ctx, ct, get_elt_from_step(step, ctx.N), key)


def hoist_rotations(context: context, ct: ciphertext, glk: galois_key, steps) -> list:
    """One ModUp of c1 shared by all rotations (src/evaluate.cu:1929-2082)."""
    if ct.size() > 2:
        raise ValueError("ciphertext size must be 2")
    if not steps:
        return []
    elts = [get_elt_from_step(s, context.N) for s in steps]
    keys = [glk.get(e) for e in elts]
    L = context.size_Ql(ct.chain_index())
    out = context._empty(len(elts), 2, L, context.N)
    context.native.hoist_rotations(ct.chain_index(), ct.data, elts, keys, out)
    return [ct._like(out[i]) for i in range(len(elts))]


def hoisting(ctx: context, ct: ciphertext, glk: galois_key, steps) -> ciphertext:
    """Sum of the rotations by `steps`: one ModUp of c1, inner products of all
    rotations accumulated, one ModDown (src/evaluate.cu:1732-1927)."""
    if ct.size() > 2:
        raise ValueError("ciphertext size must be 2")
    if not steps:
        return ct._like(ct.data.clone())
    elts = [get_elt_from_step(s, ctx.N) for s in steps]
    keys = [glk.get(e) for e in elts]
    L = ctx.size_Ql(ct.chain_index())
    out = ctx._empty(2, L, ctx.N)
    ctx.native.hoisting(ct.chain_index(), ct.data, elts, keys, out)
    return ct._like(out)


class single_chain_plaintext:
    """SingleChainPlaintext (include/single_chain_plaintext.h:37-40,
    python/src/binding.cu:405-426): a plaintext kept as its N rounded signed
    coefficients and scale, expanded to residues at the level of use.  The
    coefficients are held on the device (int64 [N])."""

    def __init__(self, coeffs, scale: float):
        self.coeffs = coeffs
        self._scale = float(scale)

    @property
    def scale(self) -> float:
        return self._scale

    @property
    def N(self) -> int:
        return int(self.coeffs.shape[0])

    @property
    def nbytes(self) -> int:
        return 8 * self.N

    def get_scale(self) -> float:
        return self._scale

    def coeffs_bytes(self) -> bytes:
        """The int64 coefficients as raw bytes (N * 8); scp_from_bytes inverts it."""
        return np.ascontiguousarray(self.coeffs.cpu().numpy(), dtype=np.int64).tobytes()


def encode_single_chain_plaintext(context: context, encoder: ckks_encoder, slots, scale: float):
    """encode_single_chain_plaintext (src/single_chain_plaintext.cu:93-150): the
    CKKS slot encoding of `slots` (complex or real) at `scale`, kept as signed
    coefficients."""
    t = _torch()
    v = np.asarray(slots)
    if v.ndim != 1:
        raise RuntimeError("encode_single_chain_plaintext: array must be 1-D")
    if len(v) > encoder.slot_count():
        raise ValueError("encode_single_chain_plaintext: too many values")
    coeffs = t.empty(context.N, dtype=t.int64, device=context.dev)
    context.native.ckks_encode_coeffs(t.from_numpy(v.astype(np.complex128)).to(context.dev), scale, coeffs)
    return single_chain_plaintext(coeffs, scale)


def scp_from_bytes(data: bytes, scale: float, N: int, context: context | None = None):
    """scp_from_bytes (python/src/binding.cu:496-519): the inverse of coeffs_bytes."""
    if len(data) != N * 8:
        raise RuntimeError(f"scp_from_bytes: byte length mismatch (got {len(data)}, expected {N * 8})")
    t = _torch()
    c = t.from_numpy(np.frombuffer(data, dtype=np.int64).copy()).to(_device(context))
    return single_chain_plaintext(c, scale)


def expand_single_chain_to_full(context: context, scp: single_chain_plaintext, target_chain_index: int):
    """expand_single_chain_to_full (src/single_chain_plaintext.cu:150-192): the
    coefficients reduced into every prime of the level, then the forward NTT."""
    if scp.N != context.N:
        raise ValueError("expand_single_chain_to_full: coeff length != N")
    L = context.size_Ql(target_chain_index)
    out = context._empty(1, L, context.N)
    context.native.expand_signed(scp.coeffs.to(context.dev).view(1, -1).contiguous(), 1, out, L)
    context.native.ntt_forward(out, 1, L, 0)
    pt = plaintext()
    pt.data, pt._chain_index, pt._scale = out[0], target_chain_index, scp.scale
    return pt


# ---------------------------------------------------------------- BSGS matvec
# Encrypted matrix-vector product by baby-step giant-step diagonals
# (include/bsgs.h, src/bsgs.cu).  y = W x for a plaintext matrix W and an
# encrypted vector x in replicated-block layout (period d_pad).
class bsgs_diagonals:
    """BsgsDiagonals (include/bsgs.h:15-21): d_pad diagonals indexed
    [g * baby_steps + b], each pre-rotated by g * baby_steps and stored as a
    level-independent plaintext of signed coefficients (SingleChainPlaintext,
    include/single_chain_plaintext.h:37-40).  Their NTT-form expansion at a
    chain index is built on first use and kept on the device (d_pad x |Ql| limbs,
    40 GiB at d_pad 4096, |Ql| 20, N 2^16), where the reference re-expands the
    plaintexts of every giant on every product (src/bsgs.cu:276-312)."""

    def __init__(self, coeffs, scale: float, d_pad: int, baby_steps: int):
        self.coeffs = coeffs  # int64 device tensor [d_pad][N]
        self.scale = float(scale)
        self.d_pad = int(d_pad)
        self.baby_steps = int(baby_steps)
        self.giant_steps = self.d_pad // self.baby_steps
        self._expanded = {}

    def expanded(self, ctx: context, chain_index: int):
        """The diagonals as NTT-form plaintexts at chain_index, in the tiled
        layout the accumulation reads (pfa_bsgs_tile_plaintexts), built once
        per level and kept on the device."""
        t = self._expanded.get(chain_index)
        if t is None:
            L = ctx.size_Ql(chain_index)
            t = ctx._empty((ctx.native.bsgs_tiled_size(chain_index, self.d_pad) + 7) // 8)
            step = min(self.d_pad, 256)
            tmp = ctx._empty(step, L, ctx.N)
            for s0 in range(0, self.d_pad, step):
                n = min(step, self.d_pad - s0)
                ctx.native.expand_signed(self.coeffs[s0:s0 + n], n, tmp[:n], L)
                ctx.native.ntt_forward(tmp[:n], n, L, 0)
                ctx.native.bsgs_tile_plaintexts(chain_index, tmp[:n], n, t, s0, self.d_pad)
            del tmp
            self._expanded[chain_index] = t
        return t

    def release(self):
        """Drop the cached expansions."""
        self._expanded.clear()

    @property
    def diagonals(self) -> list:
        """The d_pad single-chain plaintexts (views of the coefficient array)."""
        return [single_chain_plaintext(self.coeffs[d], self.scale) for d in range(self.d_pad)]


def _is_pow2(x: int) -> bool:
    return x > 0 and (x & (x - 1)) == 0


def _encode_bsgs_diagonals(context: context, encoder: ckks_encoder, rows, d_pad: int, baby_steps: int,
                           scale: float) -> bsgs_diagonals:
    """Shared tail of the pre-encoders (src/bsgs.cu:133-176, :465-513): with the
    matrix `rows` (complex, shape [num_rows][num_cols]) diag[d][t] =
    rows[t][(t + d) mod d_pad] (zero outside), diagonal g * M + b rotated right by
    g * M, tiled over the slots with period d_pad and encoded at `scale` as a
    single-chain plaintext."""
    t = _torch()
    num_rows, num_cols = rows.shape
    r = np.arange(num_rows)[:, None]
    j = (r + np.arange(d_pad)[None, :]) % d_pad  # [t][d]
    vals = np.where(j < num_cols, rows[r, np.minimum(j, num_cols - 1)], 0.0)
    diag = np.zeros((d_pad, d_pad), dtype=np.complex128)
    diag[:, :num_rows] = vals.T  # diag[d][t]
    slots = encoder.slot_count()
    coeffs = t.empty((d_pad, context.N), dtype=t.int64, device=context.dev)
    for g in range(d_pad // baby_steps):
        for b in range(baby_steps):
            d = g * baby_steps + b
            v = np.tile(np.roll(diag[d], g * baby_steps), slots // d_pad)
            context.native.ckks_encode_coeffs(t.from_numpy(v).to(context.dev), scale, coeffs[d])
    return bsgs_diagonals(coeffs, scale, d_pad, baby_steps)


def pre_encode_bsgs_diagonals(context: context, encoder: ckks_encoder, matrix, num_rows: int, num_cols: int,
                              d_pad: int, baby_steps: int, scale: float) -> bsgs_diagonals:
    """pre_encode_bsgs_diagonals (src/bsgs.cu:99-178): diag[d][t] = W[t][(t + d) mod d_pad]
    (zero outside num_rows x num_cols); diagonal g * M + b is rotated right by
    g * M, tiled over the slots with period d_pad and encoded at `scale`."""
    if num_rows == 0 or num_cols == 0:
        raise ValueError("pre_encode_bsgs_diagonals: dimensions must be non-zero")
    W = np.asarray(matrix, dtype=np.float64).ravel()
    if W.size != num_rows * num_cols:
        raise ValueError("pre_encode_bsgs_diagonals: matrix size mismatch")
    if not _is_pow2(d_pad):
        raise ValueError("pre_encode_bsgs_diagonals: d_pad must be a power of 2")
    if d_pad < num_rows or d_pad < num_cols:
        raise ValueError("pre_encode_bsgs_diagonals: d_pad must be >= max(num_rows, num_cols)")
    if baby_steps == 0 or d_pad % baby_steps:
        raise ValueError("pre_encode_bsgs_diagonals: baby_steps must divide d_pad")
    if encoder.slot_count() % d_pad:
        raise ValueError("pre_encode_bsgs_diagonals: num_slots must be multiple of d_pad")
    return _encode_bsgs_diagonals(context, encoder, W.reshape(num_rows, num_cols).astype(np.complex128), d_pad,
                                  baby_steps, scale)


class ComplexFoldMode(enum.Enum):
    """ComplexFoldMode (include/bsgs.h:81-97).  Rows: rows i and i + ceil(R/2)
    share complex row i (re(y)[i] = (W x)[i], im(y)[i] = (W x)[i + ceil(R/2)]).
    ColsConj: columns j and j + ceil(C/2) share complex column j with the second
    conjugated, for x packed as x[j] + i x[j + ceil(C/2)] (re(y) = W x)."""
    Rows = 0
    ColsConj = 1


complex_fold_mode = ComplexFoldMode  # the binding's name for the enum (binding.cu:570-572)


class complex_bsgs_diagonals:
    """ComplexBsgsDiagonals (include/bsgs.h:77-79): the same structure as
    bsgs_diagonals, with complex-folded diagonals."""

    def __init__(self, inner: bsgs_diagonals):
        self.inner = inner


def _complex_fold(W: np.ndarray, mode: ComplexFoldMode) -> np.ndarray:
    """apply_complex_fold (src/bsgs.cu:373-413): the folded complex matrix."""
    R, C = W.shape
    if mode == ComplexFoldMode.Rows:
        h = (R + 1) // 2
        out = W[:h].astype(np.complex128)
        out[:R - h] += 1j * W[h:]
        return out
    h = (C + 1) // 2
    out = W[:, :h].astype(np.complex128)
    out[:, :C - h] -= 1j * W[:, h:]
    return out


def pre_encode_bsgs_diagonals_complex(context: context, encoder: ckks_encoder, matrix, num_rows: int,
                                      num_cols: int, d_pad: int, baby_steps: int, scale: float,
                                      mode: ComplexFoldMode) -> complex_bsgs_diagonals:
    """pre_encode_bsgs_diagonals_complex (src/bsgs.cu:415-514): the matrix folded
    to complex (Rows or ColsConj), then diagonal-encoded as in the real case."""
    if num_rows == 0 or num_cols == 0:
        raise ValueError("pre_encode_bsgs_diagonals_complex: dimensions must be non-zero")
    W = np.asarray(matrix, dtype=np.float64).ravel()
    if W.size != num_rows * num_cols:
        raise ValueError("pre_encode_bsgs_diagonals_complex: matrix size mismatch")
    if not _is_pow2(d_pad):
        raise ValueError("pre_encode_bsgs_diagonals_complex: d_pad must be a power of 2")
    if baby_steps == 0 or d_pad % baby_steps:
        raise ValueError("pre_encode_bsgs_diagonals_complex: baby_steps must divide d_pad")
    folded = _complex_fold(W.reshape(num_rows, num_cols), ComplexFoldMode(mode))
    if d_pad < folded.shape[0] or d_pad < folded.shape[1]:
        raise ValueError("pre_encode_bsgs_diagonals_complex: d_pad must be >= max(folded_rows, folded_cols)")
    if encoder.slot_count() % d_pad:
        raise ValueError("pre_encode_bsgs_diagonals_complex: num_slots must be multiple of d_pad")
    return complex_bsgs_diagonals(_encode_bsgs_diagonals(context, encoder, folded, d_pad, baby_steps, scale))


def bsgs_required_steps(baby_steps: int) -> list:
    """Rotation steps the product needs (src/bsgs.cu:180-193): powers of 2
    below baby_steps (chained babies) and baby_steps (the giant stride)."""
    if baby_steps <= 1:
        return []
    steps, s = [], 1
    while s < baby_steps:
        steps.append(s)
        s <<= 1
    return steps + [baby_steps]


def compute_bsgs_babies(context: context, galois_key: galois_key, x: ciphertext, baby_steps: int) -> list:
    """babies[0] = x, babies[b] = rotate(babies[b - msb(b)], msb(b)) (src/bsgs.cu:194-214)."""
    if baby_steps == 0:
        raise ValueError("compute_bsgs_babies: baby_steps must be > 0")
    if x.size() != 2:
        raise ValueError("compute_bsgs_babies: ciphertext size must be 2")
    steps = [1 << k for k in range((baby_steps - 1).bit_length())]
    elts = [get_elt_from_step(s, context.N) for s in steps]
    if baby_steps == 1:
        return [x]
    if all(e in galois_key.keys for e in elts):
        # every rotation has its direct key: the whole chain runs in one native call
        out = context._empty(baby_steps, 2, context.size_Ql(x.chain_index()), context.N)
        context.native.bsgs_babies(x.chain_index(), x.data, baby_steps, [galois_key.get(e) for e in elts], out)
        return [x] + [x._like(out[b]) for b in range(1, baby_steps)]
    babies = [x]
    for b in range(1, baby_steps):
        bit = 1 << (b.bit_length() - 1)
        babies.append(rotate(context, babies[b - bit], bit, galois_key))
    return babies


def bsgs_apply_giants_with_babies(context: context, galois_key: galois_key, babies, diags: bsgs_diagonals):
    """bsgs_apply_giants_with_babies (src/bsgs.cu:216-357): partial_g =
    sum_b pt[g M + b] * babies[b] for every giant (one launch), then Horner
    acc = rotate(acc, M) + partial_g from g = G - 1 down to 0, one rescale, and
    the babies' scale restored."""
    M, G, d_pad = diags.baby_steps, diags.giant_steps, diags.d_pad
    if M == 0 or G == 0 or M * G != d_pad:
        raise ValueError("bsgs_apply_giants_with_babies: M*G must equal d_pad")
    if len(babies) != M:
        raise ValueError("bsgs_apply_giants_with_babies: babies size != baby_steps")
    x = babies[0]
    chain = x.chain_index()
    for c in babies:
        if c.chain_index() != chain or c.size() != 2:
            raise ValueError("babies must be size-2 ciphertexts at one chain index")
    L = context.size_Ql(chain)
    P = diags.expanded(context, chain)
    elt = get_elt_from_step(M, context.N)
    if G == 1 or elt in galois_key.keys:
        # accumulation, Horner rotations and rescale in one native call
        if L < 2:
            raise ValueError("end of modulus switching chain reached")
        out = context._empty(2, L - 1, context.N)
        context.native.bsgs_apply_giants(chain, P, [c.data for c in babies], G,
                                         galois_key.get(elt) if G > 1 else None, out)
        return x._like(out, chain=chain + 1)
    partials = context._empty(G, 2, L, context.N)
    step = 2 * L * context.N * 8  # bytes per partial ciphertext
    base_o = partials.data_ptr()
    context.native.bsgs_mac_tiled(chain, P, [c.data for c in babies], [base_o + g * step for g in range(G)])
    scale = x.scale() * diags.scale
    acc = x._like(partials[G - 1], scale=scale)
    for g in range(G - 2, -1, -1):
        acc = rotate(context, acc, M, galois_key)
        acc = add(context, acc, x._like(partials[g], scale=scale))
    acc = rescale_to_next(context, acc)
    acc.set_scale(x.scale())
    return acc


def bsgs_matmul_preencoded(context: context, galois_key: galois_key, x: ciphertext, diags: bsgs_diagonals):
    """bsgs_matmul_preencoded (src/bsgs.cu:361-368)."""
    return bsgs_apply_giants_with_babies(context, galois_key,
                                         compute_bsgs_babies(context, galois_key, x, diags.baby_steps), diags)


def bsgs_matmul_preencoded_complex(context: context, galois_key: galois_key, x: ciphertext,
                                   diags: complex_bsgs_diagonals):
    """bsgs_matmul_preencoded_complex (src/bsgs.cu:517-524): the real-path product."""
    return bsgs_matmul_preencoded(context, galois_key, x, diags.inner)


def bsgs_apply_giants_with_babies_complex(context: context, galois_key: galois_key, babies,
                                          diags: complex_bsgs_diagonals):
    """bsgs_apply_giants_with_babies_complex (src/bsgs.cu:526-532)."""
    return bsgs_apply_giants_with_babies(context, galois_key, babies, diags.inner)


# ---------------------------------------------------------------- bootstrapping
# CKKS bootstrapping with the API of include/bootstrap.h / python/src/binding.cu
# (create_bootstrap_key, bootstrap, bootstrap_required_galois_elts,
# build_c2s_diagonals, ...).  Two pipelines share ModRaise (under a transient
# sparse secret, so |I| < K), CoeffToSlot, the conjugate split into real and
# imaginary tracks, recombination and SlotToCoeff:
#   * "k28_r3" -- the reference's (src/bootstrap.cu:1703-1951) on its engine's
#     chain (ckks_engine_coeff_bits): the message scaled up to q_msg, EvalRound
#     K x - evalmod_k28_r3(x) on both tracks, then the raised ciphertext minus
#     SlotToCoeff of the rounding part, with the reference's scale-down options;
#   * "cheb63" -- this build's, on bootstrap_coeff_bits(): the message lifted to
#     q0 / 2^12 only, EvalMod as sin(2 pi x) through a degree-63 Chebyshev
#     approximation of cos(2 pi (x - 1/4) / 2^r) and r double-angle steps, and
#     SlotToCoeff of the sine times 1 / (2 pi).
# Parity is the reference's own acceptance test: decoded slots within 1e-3
# (test/ckks_engine_test.cu:182).
#
# In the "cheb63" pipeline scales are tracked exactly: diagonal plaintexts are
# encoded at the prime the following rescale drops, and every constant at the
# scale that makes the sum it joins line up, so no addition ever mixes scales.
# The reference's EvalMod snaps scales instead, and its pipeline does the same.

BOOT_K = 28            # |x| bound of EvalMod's input (|I| < K for the sparse secret)
BOOT_R = 3             # double-angle steps
BOOT_DEG = 63          # Chebyshev degree (depth 7)
BOOT_EVALMOD_LEVELS = 10
BOOT_MSG_BITS = 12     # bootstrapping lifts the message to about q0 / 2^12 first
# The transforms run at 2^b times their output scale (an exact integer multiple):
# b more bits above their rotations' key-switching noise, b fewer in the last
# layer's diagonals.  CoeffToSlot's slots (~sum |I|, hundreds) make those
# diagonals' rounding count; SlotToCoeff's slots are the small message.
BOOT_C2S_BOOST = 5
BOOT_S2C_BOOST = 10
BOOT_LT_LEVELS = 3


def bootstrap_coeff_bits(user_levels: int = 13, q0_bits: int = 60, user_bits: int = 40, s2c_bits: int = 50,
                         evalmod_bits: int = 60, c2s_bits: int = 60, special: int = 6, special_bits: int = 60,
                         eval_mod_levels: int = BOOT_EVALMOD_LEVELS):
    """Prime sizes of a bootstrappable chain for this build's EvalMod
    (create_bootstrap_key(..., evalmod="cheb63")), bottom to top, then the
    special primes: q0 | user levels | SlotToCoeff x 3 | EvalMod x 10 |
    CoeffToSlot x 3.  CoeffToSlot's diagonals are encoded at the scale of the
    prime its rescale drops and act on slots of size ~sum |I| (hundreds to
    thousands), so its primes are the widest; SlotToCoeff acts on the small
    refreshed message."""
    return ([q0_bits] + [user_bits] * user_levels + [s2c_bits] * BOOT_LT_LEVELS + [evalmod_bits] * eval_mod_levels
            + [c2s_bits] * BOOT_LT_LEVELS + [special_bits] * special)


def ckks_engine_coeff_bits(num_scale_levels: int = 14, num_special_primes: int = 6) -> list:
    """The reference engine's bootstrappable chain (src/ckks_engine.cu:117-126,
    its default CKKSEngineConfig: 14 scale levels, 6 special primes, |Q| = 30,
    dnum = 5), bottom to top, then the special primes:
        q_msg 58 | scale 40 x num_scale_levels | SlotToCoeff 58 x 3 |
        EvalRound 58 x 9 | CoeffToSlot 29 x 3 | special 58 x num_special_primes.
    The chain of create_bootstrap_key(..., eval_mod_levels=9) (evalmod "k28_r3")."""
    if num_scale_levels < 2 or num_special_primes < 1:
        raise ValueError("need at least 2 scale levels and 1 special prime")
    if (16 + num_scale_levels) % num_special_primes:
        raise ValueError("size_Q must be divisible by num_special_primes")
    return ([58] + [40] * num_scale_levels + [58] * BOOT_LT_LEVELS + [58] * 9 + [29] * BOOT_LT_LEVELS
            + [58] * num_special_primes)


def _brv_index(x: int, bits: int) -> int:
    r = 0
    for _ in range(bits):
        r = (r << 1) | (x & 1)
        x >>= 1
    return r


def _fft_stages(N: int, inverse: bool):
    """The special FFT z = B_L ... B_1 P u (z_j = sum_k u_k zeta^(5^j k), P the
    bit reversal) as butterfly stages B_s (or their inverses), each a dict
    offset -> diagonal (entry (r, r + offset))."""
    n, M = N // 2, 2 * N
    rot = np.array([pow(5, j, M) for j in range(n)], dtype=np.int64)
    out = []
    length = 2
    while length <= n:
        lenh, lenq = length // 2, length * 4
        j = np.arange(lenh)
        w = np.exp(1j * np.pi * ((rot[j] % lenq) * (M // lenq)) / N)
        top = (np.arange(0, n, length)[:, None] + j[None, :]).ravel()
        wt = np.tile(w, n // length)
        d0 = np.zeros(n, complex)
        dp = np.zeros(n, complex)
        dm = np.zeros(n, complex)
        if not inverse:   # out[t] = in[t] + w in[t+h]; out[t+h] = in[t] - w in[t+h]
            d0[top], dp[top], d0[top + lenh], dm[top + lenh] = 1, wt, -wt, 1
        else:             # in[t] = (out[t] + out[t+h]) / 2; in[t+h] = (out[t] - out[t+h]) / (2 w)
            d0[top], dp[top], d0[top + lenh], dm[top + lenh] = 0.5, 0.5, -0.5 / wt, 0.5 / wt
        st = {0: d0, lenh: dp}
        st[n - lenh] = st.get(n - lenh, 0) + dm  # the last stage's +-n/2 diagonals coincide
        out.append(st)
        length <<= 1
    return out


def _diag_product(A, B, n):
    """(A B) from diagonal forms: (A B)[r][r+d] = sum A_d1[r] B_d2[r + d1], d = d1 + d2 mod n."""
    C = {}
    for d1, a in A.items():
        for d2, b in B.items():
            d = (d1 + d2) % n
            C[d] = C.get(d, 0) + a * np.roll(b, -d1)
    return {d: v for d, v in C.items() if np.max(np.abs(v)) > 1e-300}


class _LTLayers:
    """LinearTransformDiagonals (include/bootstrap.h): per layer, diagonals
    {offset: values} of the product of its butterfly stages, the stage unit
    2^s0 and the baby-step count."""

    def __init__(self, log_n: int, stages_per_layer, inverse: bool):
        N = 1 << log_n
        n = N // 2
        logn = n.bit_length() - 1
        if sum(stages_per_layer) != logn:
            raise ValueError(f"stages_per_layer must sum to log2(slots) = {logn}")
        st = _fft_stages(N, inverse)
        if inverse:   # CoeffToSlot applies B_L^-1 first
            st = st[::-1]
        self.N, self.n, self.layers, self.units = N, n, [], []
        k = 0
        for g in stages_per_layer:
            L = {0: np.ones(n, complex)}
            for s in st[k:k + g]:
                L = _diag_product(s, L, n)
            lo = k if not inverse else logn - k - g  # lowest stage index of the layer
            self.layers.append(L)
            self.units.append(1 << lo)
            k += g
        self.stages_per_layer = list(stages_per_layer)

    def baby_giant(self, i):
        """(n1, {giant: [(baby, offset)]}) of layer i, offsets in units of 2^s0.
        n1 is the smallest power of two with n1^2 >= the layer's diagonal
        count (8 for 5 stages: 7 baby and 7 giant rotations).  The reference
        takes n1 = 2^(s-1) (src/bootstrap.cu:323: 15 babies, 3 giants); with
        this library's hoisted babies and batched giants that split measured
        slower (config 5: 27.7 -> 29.5 ms, EvalRound 26.5 -> 28.7 ms, 53
        instead of 39 Galois keys)."""
        unit, n = self.units[i], self.n
        e = sorted(d // unit for d in self.layers[i])
        span = n // unit
        n1 = 1
        while n1 * n1 < len(e):
            n1 <<= 1
        groups = {}
        for x in e:
            g, b = divmod(x, n1)
            groups.setdefault(g, []).append((b, x * unit))
        return n1, groups, span

    def rotation_steps(self):
        steps = set()
        for i in range(len(self.layers)):
            n1, groups, span = self.baby_giant(i)
            unit = self.units[i]
            for g, terms in groups.items():
                for b, _ in terms:
                    if b:
                        steps.add(b * unit)
                if g:
                    steps.add(_signed_step(g * n1 * unit, self.n))
        return sorted(steps)


def _signed_step(step: int, n: int) -> int:
    step %= n
    return step - n if step > n // 2 else step


def build_c2s_diagonals(log_n: int, stages_per_layer=(5, 5, 5)) -> _LTLayers:
    """CoeffToSlot as layered butterflies (src/bootstrap.cu:256-387): slots ->
    the packed coefficients u_k = m_k + i m_(k+N/2), in bit-reversed order."""
    return _LTLayers(log_n, stages_per_layer, True)


def build_s2c_diagonals(log_n: int, stages_per_layer=(5, 5, 5)) -> _LTLayers:
    """SlotToCoeff (src/bootstrap.cu:389-437): the inverse of CoeffToSlot."""
    return _LTLayers(log_n, stages_per_layer, False)


def c2s_required_rotation_steps(diags: _LTLayers, num_slots: int) -> list:
    return diags.rotation_steps()


def bootstrap_required_galois_elts(log_n: int, stages_per_layer=(5, 5, 5)) -> list:
    """Galois elements of the CoeffToSlot and SlotToCoeff rotations plus
    conjugation (python/src/binding.cu:301-318)."""
    N = 1 << log_n
    steps = sorted(set(build_c2s_diagonals(log_n, stages_per_layer).rotation_steps())
                   | set(build_s2c_diagonals(log_n, stages_per_layer).rotation_steps()))
    return get_elts_from_steps(steps, N) + [2 * N - 1]


def _default_stages(log_n: int):
    logn = log_n - 1
    return [logn // 3 + (1 if i < logn % 3 else 0) for i in range(3)]


def _const_plain(ctx: context, value: complex, scale: float, chain: int) -> plaintext:
    """The constant `value` in every slot, exactly: coefficient 0 = Re(value) scale
    and coefficient N/2 = Im(value) scale (X^(N/2) is i at every slot).  A real
    constant is the same residue at every NTT point, so it is written directly."""
    value = complex(value)
    L = ctx.size_Ql(chain)
    pt = plaintext()
    pt._chain_index, pt._scale = chain, float(scale)
    re = int(round(value.real * scale))
    im = int(round(value.imag * scale))
    def make():
        if im == 0:
            r = np.array([re % q for q in ctx.moduli[:L]], dtype=np.uint64)
            return _to_dev(r, ctx.dev).view(L, 1).expand(L, ctx.N).contiguous()
        c = np.zeros(ctx.N, dtype=np.int64)
        c[0] = re
        c[ctx.N // 2] = im
        return ctx._ntt(ctx._signed_to_rns(c, L), L)

    pt.data = ctx._cached_const(("const", re, im, L), make)
    return pt


class small_bootstrap_key:
    """SmallBootstrapKey (include/bootstrap.h): the key-switching pair that
    moves a ciphertext from the user's dense secret to a transient sparse one
    (ksk_to_sparse) and back (ksk_to_dense)."""

    def __init__(self, ksk_to_sparse=None, ksk_to_dense=None):
        self.ksk_to_sparse = ksk_to_sparse
        self.ksk_to_dense = ksk_to_dense


def _small_bootstrap_key(context: context, dense_sk: secret_key, sparse_hamming_weight: int, seed=None):
    if sparse_hamming_weight <= 0:
        raise ValueError("create_small_bootstrap_key: hamming_weight must be > 0")
    dense_sk._require()
    rng = _rng(seed)
    sparse = secret_key().generate_sparse(context, sparse_hamming_weight, seed=rng)
    small = small_bootstrap_key(relin_key(sparse._kswitch_key(context, dense_sk.sk, rng)),
                                relin_key(dense_sk._kswitch_key(context, sparse.sk, rng)))
    return small, sparse


def create_small_bootstrap_key(context: context, dense_sk: secret_key, sparse_hamming_weight: int = 128,
                               seed=None) -> small_bootstrap_key:
    """create_small_bootstrap_key (src/bootstrap.cu:185-202): the sparse
    secret exists only inside this call."""
    return _small_bootstrap_key(context, dense_sk, sparse_hamming_weight, seed)[0]


def apply_kswitch(context: context, ct: ciphertext, key: relin_key) -> ciphertext:
    """apply_kswitch_inplace: (c0, c1) under s -> under the key's target secret
    (the Galois path with the identity element 1)."""
    return _apply_galois_key(context, ct, 1, key.data)


class bootstrap_key:
    """BootstrapKey (include/bootstrap.h): the encapsulation pair, the Galois
    keys of CoeffToSlot, SlotToCoeff and conjugation, the relinearization
    key, and the layers' diagonal plaintexts, encoded at the levels they are
    applied at."""

    def __init__(self):
        self.small = None
        self.glk = None
        self.rlk = None
        self.c2s = None
        self.s2c = None
        self.c2s_pts = []   # per layer: a _LayerPlan
        self.s2c_pts = []
        self.cheb = None
        self.K, self.r = BOOT_K, BOOT_R
        # "k28_r3": the reference's pipeline (EvalRound with evalmod_k28_r3,
        # then saved - SlotToCoeff(round)); "cheb63": this build's EvalMod
        # (sin(2 pi x) by a degree-63 Chebyshev fit, SlotToCoeff of the sine)
        self.evalmod = "cheb63"
        self.eval_mod_levels = BOOT_EVALMOD_LEVELS
        self.user_scale = 0.0
        self.split_scale_down = False
        self.s2c_start = 0   # chain index of SlotToCoeff's first layer
        self.c2s_boost, self.s2c_boost = BOOT_C2S_BOOST, BOOT_S2C_BOOST


class _LayerPlan:
    """One transform layer, ready for the BSGS accumulation: the baby offsets b
    (in units), the giant indices g, the diagonal plaintexts as a [G][M] grid
    (a shared zero plaintext where (g, b) has no diagonal), and the same grid
    in the accumulation's tiled layout (pfa_bsgs_tile_plaintexts: each work
    item's plaintexts contiguous, limbs below 2^40 in 5 bytes a residue),
    which the accumulation reads."""

    def __init__(self, babies, giants, grid, scale, zero, tiled=None):
        self.babies, self.giants, self.grid, self.scale, self.zero = babies, giants, grid, scale, zero
        self.tiled = tiled


def _encode_layer(ctx, enc, lt: _LTLayers, i: int, chain: int, factor: complex, scale_div: int = 1,
                  encode_scale: float = 0.0) -> _LayerPlan:
    """Layer i's diagonals, each pre-rotated by minus its giant step, encoded
    at `chain` with the scale of the prime the following rescale drops (or
    encode_scale when given), divided by scale_div (a power of two, so the
    scale stays exact)."""
    n1, groups, span = lt.baby_giant(i)
    L = ctx.size_Ql(chain)
    scale = (float(encode_scale) if encode_scale > 0 else float(ctx.moduli[L - 1])) / scale_div
    babies = sorted({b for terms in groups.values() for b, _ in terms})
    giants = sorted(groups)
    zero = None
    grid = []
    for g in giants:
        shift = g * n1 * lt.units[i]
        have = {b: d for b, d in groups[g]}
        for b in babies:
            if b in have:
                v = np.roll(lt.layers[i][have[b] % lt.n] * factor, shift)
                grid.append(enc.encode_complex_vector(ctx, v, scale, chain).data)
            else:
                if zero is None:
                    zero = ctx._empty(L, ctx.N).zero_()
                grid.append(zero)
    D = len(grid)
    tiled = ctx._empty((ctx.native.bsgs_tiled_size(chain, D) + 7) // 8)
    for d, pt in enumerate(grid):
        ctx.native.bsgs_tile_plaintexts(chain, pt, 1, tiled, d, D)
    return _LayerPlan(babies, giants, grid, scale, zero, tiled)


BOOT_EVALMODS = ("k28_r3", "cheb63")


def create_bootstrap_key(context: context, encoder: ckks_encoder, dense_sk: secret_key,
                         sparse_hamming_weight: int = 128, eval_mod_levels: int = 0, user_scale: float = 0.0,
                         split_scale_down: bool = False, stages_per_layer=None, seed=None,
                         evalmod: str = "k28_r3") -> bootstrap_key:
    """create_bootstrap_key (src/bootstrap.cu:895-980, python/src/binding.cu:320-327).
    The context must carry bootstrap_required_galois_elts.  The ModRaise runs
    under a transient sparse secret of weight sparse_hamming_weight; the
    rotation and relinearization keys are the dense secret's.

    evalmod "k28_r3" (default) is the reference's pipeline: CoeffToSlot on
    chains 1 .. 3 (normalized by 1 / (2 K), K = 28, when eval_mod_levels > 0,
    by 1 otherwise), SlotToCoeff from chain 4 + eval_mod_levels with its last
    layer encoded at user_scale when user_scale > 0 and not split_scale_down.
    eval_mod_levels = 0 is the reference's round-trip key (CoeffToSlot straight
    into SlotToCoeff; bootstrap() then refuses it, as the reference does); a
    full bootstrap needs at least 9 (evalmod_k28_r3), the chain of
    ckks_engine_coeff_bits.

    evalmod "cheb63" is this build's pipeline (bootstrap_coeff_bits chain):
    EvalMod by a degree-63 Chebyshev fit over 10 levels; eval_mod_levels must
    be 0 or 10, user_scale 0 and split_scale_down false (it returns the
    message at the input scale)."""
    if evalmod not in BOOT_EVALMODS:
        raise ValueError(f"evalmod must be one of {BOOT_EVALMODS}")
    if eval_mod_levels < 0:
        raise ValueError("eval_mod_levels must be >= 0")
    if evalmod == "cheb63":
        if eval_mod_levels not in (0, BOOT_EVALMOD_LEVELS):
            raise ValueError(f"evalmod 'cheb63' takes {BOOT_EVALMOD_LEVELS} levels")
        if user_scale != 0.0 or split_scale_down:
            raise ValueError("evalmod 'cheb63' bootstraps at the ciphertext's own scale "
                             "(user_scale and split_scale_down do not apply)")
        eval_mod_levels = BOOT_EVALMOD_LEVELS
    if user_scale < 0.0:
        raise ValueError("user_scale must be >= 0")
    ctx, enc = context, encoder
    log_n = ctx.N.bit_length() - 1
    stages = list(stages_per_layer or _default_stages(log_n))
    nl = len(stages)
    need = 2 * nl + eval_mod_levels + 1
    if ctx.size_Q < need:
        raise ValueError(f"bootstrapping needs at least {need} primes")
    missing = [e for e in bootstrap_required_galois_elts(log_n, stages) if e not in ctx.galois_elts]
    if missing:
        raise ValueError("the context's galois_elts lack bootstrap_required_galois_elts")
    rng = _rng(seed)
    bk = bootstrap_key()
    bk.evalmod, bk.eval_mod_levels = evalmod, eval_mod_levels
    bk.user_scale, bk.split_scale_down = float(user_scale), bool(split_scale_down)
    bk.small = _small_bootstrap_key(ctx, dense_sk, sparse_hamming_weight, rng)[0]
    bk.rlk = dense_sk.gen_relinkey(ctx, seed=rng)
    bk.glk = galois_key(ctx.galois_elts)
    for elt in bootstrap_required_galois_elts(log_n, stages):
        bk.glk.keys[elt] = dense_sk._galois_key_for(ctx, elt, rng)
    bk.c2s = build_c2s_diagonals(log_n, stages)
    bk.s2c = build_s2c_diagonals(log_n, stages)
    # The transforms run 2^boost above their output scale (an exact integer
    # multiple taken back out in their last layer's diagonals).  On narrow
    # CoeffToSlot primes (the reference engine's 29-bit ones) the diagonals'
    # rounding dominates instead, so no boost there.
    c2s_prime_bits = ctx.moduli[ctx.size_Ql(1) - 1].bit_length()
    bk.c2s_boost = BOOT_C2S_BOOST if c2s_prime_bits > 40 else 0
    bk.s2c_boost = BOOT_S2C_BOOST
    # CoeffToSlot at chains 1 .. nl with 1 / (2K) in its last layer (1 for the
    # round-trip key); SlotToCoeff after EvalMod, with 1 / (2 pi) in its first
    # layer for this build's sine (the reference's EvalRound needs none)
    c2s_norm = 1 / (2 * BOOT_K) if eval_mod_levels > 0 else 1.0
    bk.c2s_pts = [_encode_layer(ctx, enc, bk.c2s, i, 1 + i, c2s_norm if i == nl - 1 else 1.0,
                                1 << bk.c2s_boost if i == nl - 1 else 1)
                  for i in range(nl)]
    bk.s2c_start = 1 + nl + eval_mod_levels
    s2c_first = 1 / (2 * np.pi) if evalmod == "cheb63" else 1.0
    last_scale = bk.user_scale if (evalmod == "k28_r3" and not bk.split_scale_down) else 0.0
    bk.s2c_pts = [_encode_layer(ctx, enc, bk.s2c, i, bk.s2c_start + i, s2c_first if i == 0 else 1.0,
                                1 << bk.s2c_boost if i == nl - 1 else 1, last_scale if i == nl - 1 else 0.0)
                  for i in range(nl)]
    if evalmod == "cheb63":
        bk.cheb = evalmod_chebyshev(BOOT_K, BOOT_R, BOOT_DEG)
    return bk


def _apply_layer(ctx, ct: ciphertext, lt: _LTLayers, pts, i: int, glk, rescale: bool = True) -> ciphertext:
    """sum_d D_d . rot(ct, d) by baby steps (hoisted rotations) and giant steps:
    one pfa_bsgs_mac forms every giant's sum of diagonal x baby products, the
    giant rotations follow.  The giant rotations and the sum run before the
    one rescale, where the scale is q_drop times larger and their
    key-switching noise q_drop times smaller next to it."""
    plan = pts[i]
    n1, _, _ = lt.baby_giant(i)
    unit = lt.units[i]
    rotated = {0: ct}
    steps = [b * unit for b in plan.babies if b]
    if steps:
        for b, r in zip([b for b in plan.babies if b], hoist_rotations(ctx, ct, glk, steps)):
            rotated[b] = r
    L = ctx.size_Ql(ct.chain_index())
    parts = ctx._empty(len(plan.giants), 2, L, ctx.N)
    ctx.native.bsgs_mac_tiled(ct.chain_index(), plan.tiled, [rotated[b].data for b in plan.babies],
                        [parts[k] for k in range(len(plan.giants))])
    # the giants' rotations are independent: one batched rotation (each part
    # its own element and key) when every key is present, then one weighted
    # sum of all parts (weights 1; the same residues as the pairwise adds)
    scale = ct.scale() * plan.scale
    moved = [k for k, g in enumerate(plan.giants) if g]
    elts = [get_elt_from_step(_signed_step(plan.giants[k] * n1 * unit, lt.n), ctx.N) for k in moved]
    if moved and all(e in glk.keys for e in elts):
        rot = ctx._empty(len(moved), 2, L, ctx.N)
        src = parts[moved[0]:moved[-1] + 1] if moved == list(range(moved[0], moved[-1] + 1)) else \
            parts[moved].contiguous()
        ctx.native.rotate_batch(ct.chain_index(), src.contiguous(), elts, [glk.keys[e] for e in elts], rot)
        terms = [parts[k] for k, g in enumerate(plan.giants) if not g] + [rot[i] for i in range(len(moved))]
    else:
        terms = []
        for k, g in enumerate(plan.giants):
            part = ct._like(parts[k], scale=scale)
            terms.append((rotate(ctx, part, _signed_step(g * n1 * unit, lt.n), glk) if g else part).data)
    acc, i = None, 0
    while i < len(terms):  # pfa_ct_lincomb takes up to 8 inputs
        chunk = terms[i:i + 8] if acc is None else [acc.data] + terms[i:i + 7]
        i += len(chunk) if acc is None else len(chunk) - 1
        out = ctx._empty(2, L, ctx.N)
        ctx.native.ct_lincomb(L, chunk, [1] * len(chunk), out)
        acc = ct._like(out, scale=scale)
    return rescale_to_next(ctx, acc) if rescale else acc


def _boosted(ctx, ct: ciphertext, bits: int) -> ciphertext:
    """ct times the integer 2^bits, read at 2^bits its scale: the same message,
    with the noise a transform adds that much smaller next to it."""
    out = multiply_plain(ctx, ct, _const_plain(ctx, 1 << bits, 1.0, ct.chain_index()))
    out.set_scale(ct.scale() * (1 << bits))
    return out


def _transform(ctx, ct, lt, pts, glk, boost, last_rescale=True):
    ct = _boosted(ctx, ct, boost)
    nl = len(lt.layers)
    for i in range(nl):
        ct = _apply_layer(ctx, ct, lt, pts, i, glk, rescale=last_rescale or i < nl - 1)
    return ct


def apply_c2s_inplace(context: context, ct: ciphertext, bk: bootstrap_key) -> ciphertext:
    """CoeffToSlot (src/bootstrap.cu apply_c2s_inplace): slots -> the packed
    coefficients in bit-reversed order, times 1 / (2K) (1 for a round-trip
    key), at ct's scale."""
    return _transform(context, ct, bk.c2s, bk.c2s_pts, bk.glk, bk.c2s_boost)


def apply_s2c_inplace(context: context, ct: ciphertext, bk: bootstrap_key) -> ciphertext:
    """SlotToCoeff (src/bootstrap.cu apply_s2c_inplace): the inverse layout
    change (times 1 / (2 pi) for the "cheb63" key), at ct's scale, or at
    user_scale when the key bakes it into the last layer."""
    return _transform(context, ct, bk.s2c, bk.s2c_pts, bk.glk, bk.s2c_boost)


def mod_raise_inplace(context: context, ct: ciphertext, bk) -> ciphertext:
    """mod_raise_inplace (src/bootstrap.cu:204-215): a ciphertext (brought to the
    bottom of the chain first) is switched to the sparse secret, each residue
    mod q0 lifted centred into every prime of chain index 1 (pfa_mod_raise),
    and switched back to the dense secret.  bk is a small_bootstrap_key or a
    bootstrap_key.  Returns the raised ciphertext (chain index 1)."""
    small = bk.small if isinstance(bk, bootstrap_key) else bk
    bottom = context.size_Q
    if ct.chain_index() != bottom:
        ct = mod_switch_to(context, ct, bottom)
    ct = apply_kswitch(context, ct, small.ksk_to_sparse)
    out = context._empty(ct.size(), context.size_Q, context.N)
    context.native.mod_raise(ct.data, out)
    return apply_kswitch(context, ct._like(out, chain=1), small.ksk_to_dense)


def evalmod_chebyshev(K: int = BOOT_K, r: int = BOOT_R, deg: int = BOOT_DEG) -> np.ndarray:
    """Chebyshev coefficients (interpolation at the deg + 1 Chebyshev nodes) of
    cos(2 pi (K t - 1/4) / 2^r) on [-1, 1]; r double angles c <- 2 c^2 - 1 then
    give sin(2 pi K t) (the role of src/evalmod.cu's EvalRound tables)."""
    from numpy.polynomial import chebyshev as _C

    k = np.arange(deg + 1)
    nodes = np.cos(np.pi * (k + 0.5) / (deg + 1))
    return _C.chebfit(nodes, np.cos(2 * np.pi * (K * nodes - 0.25) / 2 ** r), deg)


def _cheb_split(c):
    """p = sum c_j T_j of degree d >= 8 as T_m hi + lo, m the largest power of two
    <= d (T_(m+i) = 2 T_m T_i - T_(m-i)); returns (m, hi, lo)."""
    deg = len(c) - 1
    m = 1 << (deg.bit_length() - 1)
    hi = [c[m]] + [2 * c[m + i] for i in range(1, deg - m + 1)]
    lo = [c[i] - (c[2 * m - i] if 2 * m - i <= deg else 0.0) for i in range(m)]
    return m, hi, lo


def _cheb_depth(deg: int) -> int:
    """Levels the evaluation in _eval_mod consumes for a degree-deg polynomial."""
    if deg < 8:
        return max(1, (deg - 1).bit_length() + 1)
    m = 1 << (deg.bit_length() - 1)
    return max(_cheb_depth(deg - m) + 1, m.bit_length(), _cheb_depth(m - 1))


class _GpuEngine:
    """The ciphertext operations both EvalMod families are written over, run by
    the native library: mod_switch_to, a weighted sum with integer weights
    (pfa_ct_lincomb), multiply_and_relin (with and without the rescale),
    rescale_to_next and add.  The test suite runs the same EvalMod code over
    an oracle implementation of these operations and compares residues."""

    def __init__(self, ctx, rlk):
        self.ctx, self.rlk = ctx, rlk

    def size_Ql(self, chain: int) -> int:
        return self.ctx.size_Ql(chain)

    def prime(self, i: int) -> int:
        return self.ctx.moduli[i]

    def to(self, a, chain: int):
        return mod_switch_to(self.ctx, a, chain)

    def lincomb(self, terms, bias, chain: int, scale: float, like):
        """sum_t k_t a_t (+ bias on poly 0 of each member) over the first
        size_Ql(chain) limbs of every input, as a ciphertext like `like` at
        chain and scale; the k_t are Python ints in int64 range, bias a Python
        int or None."""
        L = self.ctx.size_Ql(chain)
        out = self.ctx._empty(like.size(), L, self.ctx.N)
        _ct_lincomb(self.ctx, L, [a.data for a, _ in terms], [k for _, k in terms], out, bias, like._members)
        return like._like(out, chain=chain, scale=scale)

    def mul_relin(self, a, b):
        return multiply_and_relin(self.ctx, a, b, self.rlk)

    def mul_relin_rescale(self, a, b):
        return multiply_and_relin_rescale(self.ctx, a, b, self.rlk)

    def rescale(self, a):
        return rescale_to_next(self.ctx, a)

    def add(self, a, b):
        return add(self.ctx, a, b)


def _eval_mod(ctx, ct: ciphertext, bk: bootstrap_key) -> ciphertext:
    """cos(2 pi (K t - 1/4) / 2^r) by Chebyshev (Paterson-Stockmeyer splitting at
    powers of two, src/evalmod.cu:196-335 for the pattern), then r double
    angles: sin(2 pi K t) for t in [-1, 1]."""
    return _eval_mod_cheb(_GpuEngine(ctx, bk.rlk), ct, list(bk.cheb), bk.r)


def _eval_mod_cheb(eng, ct, cheb, r: int):
    """_eval_mod's operation sequence over an engine (see _GpuEngine).

    Every weighted sum is one lincomb over the Chebyshev terms at their own
    levels, with the integer weights round(c_j S q / scale_j) that land it at
    the exact scale S q, followed by one rescale to S: scales never drift and
    no addition mixes them.  T_k = 2 T_a T_b - T_1 and 2 y^2 - 1 are formed the
    same way before their rescale."""
    T = {1: ct}

    def q_drop(chain):
        return eng.prime(eng.size_Ql(chain) - 1)

    def lincomb(terms, bias, chain, scale):
        for _, k in terms:
            if not -(1 << 63) <= k < (1 << 63):
                raise ValueError("Chebyshev weight outside int64")
        return eng.lincomb(terms, bias, chain, scale, ct)

    def product(a, b):
        c = max(a.chain_index(), b.chain_index())
        return eng.mul_relin(eng.to(a, c), eng.to(b, c))

    def cheb_T(k):
        if k in T:
            return T[k]
        if k % 2 == 0:
            p = product(cheb_T(k // 2), cheb_T(k // 2))
            pre = lincomb([(p, 2)], -round(p.scale()), p.chain_index(), p.scale())
        else:
            p = product(cheb_T((k + 1) // 2), cheb_T((k - 1) // 2))
            t1 = cheb_T(1)
            pre = lincomb([(p, 2), (t1, -round(p.scale() / t1.scale()))], None, p.chain_index(), p.scale())
        T[k] = eng.rescale(pre)
        return T[k]

    def evaluate(c, target_scale, target_chain):
        deg = len(c) - 1
        chain = target_chain - 1
        q = q_drop(chain)
        if deg < 8:
            terms = []
            for j in range(1, deg + 1):
                if c[j] != 0.0:
                    t = cheb_T(j)
                    terms.append((t, round(c[j] * target_scale * q / t.scale())))
            pre = lincomb(terms, round(c[0] * target_scale * q), chain, target_scale * q)
            res = eng.rescale(pre)
            res.set_scale(target_scale)
            return res
        m, hi, lo = _cheb_split(c)
        Tm = eng.to(cheb_T(m), chain)
        hi_ct = evaluate(hi, target_scale * q / Tm.scale(), chain)
        prod = eng.mul_relin_rescale(Tm, hi_ct)
        prod.set_scale(target_scale)
        return eng.add(prod, evaluate(lo, target_scale, target_chain))

    y = evaluate(list(cheb), ct.scale(), ct.chain_index() + _cheb_depth(len(cheb) - 1))
    for _ in range(r):
        p = product(y, y)
        y = eng.rescale(lincomb([(p, 2)], -round(p.scale()), p.chain_index(), p.scale()))
    return y


# ---------------------------------------------------------------- the reference's EvalMod
# evalmod_k7_r3 / evalmod_k16_r3 / evalmod_k28_r3 / evalmod_k28_r4
# (include/evalmod.h, src/evalmod.cu): sin(2 pi K x) / (2 pi) for x in
# [-1, 1] as a Chebyshev-basis polynomial for (2 pi)^(-1/2^R) cos(2 pi K x / 2^R
# - pi / 2^(R+1)) followed by R double-angle steps y <- 2 y^2 - (2 pi)^(-2^(j-R)).
# The operation order is the reference's: the Chebyshev basis by T_2n = 2 T_n^2
# - 1 and T_(a+b) = 2 T_a T_b - T_(a-b) with the same level alignment, weighted
# sums with one deferred rescale, the same Paterson-Stockmeyer factorings, and
# the scale of every rescaled result set back to the input's ("snapped": the
# dropped prime is taken to equal the scale).  A weighted sum of ciphertexts by
# constants is one pfa_ct_lincomb with the integer weights round(c scale) -- the
# residues of the reference's multiply_plain-by-constant then add sequence.
#
# The coefficient tables define the polynomials and are kept equal to the
# reference's (src/evalmod.cu:25-47 K = 7, :57-77 K = 16, :90-120 K = 28).

_K7_LOW = (-5.92365525763352552e-03, -1.05915002790352347e-01, 1.81872438169629558e-01,
           -7.96115559593863209e-02, 6.18237166588616383e-01, 9.97204899504430670e-02,
           -2.85567102345358925e-01, -3.02985739088491718e-02, 5.23393518416412837e-02)
_K7_HIGH = (0.0, 3.49656797384041707e-03, -5.21322493828673197e-03, -2.75767647883437550e-04,
            3.34517473917776004e-04, 1.47041114332627232e-05, -1.50752826718614230e-05,
            -5.67939380614890243e-07)
# degree 31, K = 16: entry 0 of each the constant, 1 .. 7 those of T_1 .. T_7
_K16_Q_HIGH = (1.40933240904887619e-05, 1.50639230276274228e-06, -1.94594040092296340e-06,
               -9.53210705782742233e-08, 1.13318833226784231e-07, 5.12709912705527410e-09,
               -5.64857600334760771e-09, -2.37565221374504097e-10)
_K16_Q_LOW = (3.59519354992413262e-02, 6.20731655651990660e-03, -1.25289184971230146e-02,
              -9.32191173092421330e-04, 1.64251931763363971e-03, 1.07868728320514593e-04,
              -1.68130129335233066e-04, -1.07079565087396969e-05)
_K16_R_HIGH = (-1.03480520058724892e-01, 9.00051357854676909e-02, -8.54845145538975948e-01,
               -1.80792080525974813e-01, 7.33614949409451600e-01, 9.95683206882135990e-02,
               -2.78190804126826174e-01, -3.64211934038645019e-02)
_K16_R_LOW = (1.22772867008426184e-01, -2.97084681220240107e-02, 4.22982423883966452e-01,
              -7.97287003613950523e-02, -1.10422768440682217e-02, 1.05502625978328088e-01,
              7.22752525999589279e-01, 2.62006578429296658e-02)
# degree 49, K = 28: coefficient 0 the constant, 1 .. 7 those of T_1 .. T_7
_K28_AUX = (-0.4674215360340989, -0.24807246365084598, -0.03360736343811264, 0.10485552200765141,
            0.012171628025753911, -0.031034212401993305, -0.003985828764410408, 0.0)
_K28_QUOT = ((-0.7500012154934053, 4.148627473785995e-06, 2.707983311367457e-07, -4.324538856989888e-07,
              -2.648274421485692e-08, 3.9515438249932484e-08, 2.4720260690299275e-09, 0.0),
             (-6.511205244110998e-09, -7.076428529570776e-10, 1.0183620860162692e-09, 0.0, 0.0, 0.0, 0.0, 4.0),
             (0.007868944223231958, 0.0014193060148561195, -0.003081157124604844, -0.00025275745577540515,
              0.0005030348400875631, 3.734766164626263e-05, -7.780382338014487e-05, 1.0))
_K28_REM = ((-1.1324455480972702, -0.8116709016985189, -0.20294197180913795, 0.5290215620326779,
             -0.32084902738708476, 0.43458317383580536, -0.06303880005650665, 0.0),
            (0.23316927298939902, 0.12938749185636858, -0.3042902283756468, -0.008967445477730096,
             -0.6955791340472846, -0.07562064123442451, 1.2510854562849574, 2.0),
            (0.1429148264191405, 0.4544397978460022, -0.8401926425765848, -0.4292803758141986,
             -1.495563076527614, 0.3580084476476745, 1.7971594278092713, 1.0))

EVALMOD_K = {"k7_r3": 7, "k16_r3": 16, "k28_r3": 28, "k28_r4": 28}
EVALMOD_R = {"k7_r3": 3, "k16_r3": 3, "k28_r3": 3, "k28_r4": 4}
# levels consumed: basis (3) + the variant's products, then R double angles
EVALMOD_LEVELS = {"k7_r3": 8, "k16_r3": 9, "k28_r3": 9, "k28_r4": 10}


def _ct_lincomb(ctx, L: int, ins, consts, out, bias, members: int = 1) -> None:
    """pfa_ct_lincomb on plain ciphertexts or bundles (one call; the bias goes
    to poly 0 of every member)."""
    ctx.native.ct_lincomb(L, ins, consts, out, bias, ct_size=None if members == 1 else 2)


def _bundle(ctx, cts) -> ciphertext:
    """Size-2 ciphertexts at one level and scale -> one bundle (their data stacked)."""
    c0 = cts[0]
    for c in cts:
        if c.size() != 2 or c._members != 1 or c.chain_index() != c0.chain_index():
            raise ValueError("bundle members must be size-2 ciphertexts at one level")
        _check_scale(c, c0)
    # copied with the library's streaming copy: a torch kernel between the
    # library's launches on torch's default stream costs far more than the copy
    data = ctx._empty(2 * len(cts), *c0.data.shape[1:])
    for i, c in enumerate(cts):
        _N.stream_copy(data[2 * i:2 * i + 2], c.data.contiguous())
    b = c0._like(data)
    b._members = len(cts)
    return b


def _unbundle(b: ciphertext) -> list:
    out = []
    for m in range(b._members):
        c = b._like(b.data[2 * m:2 * m + 2].contiguous())
        c._members = 1
        out.append(c)
    return out


class _EvalModOps:
    """The reference's EvalMod operations on ciphertexts through an engine (see
    _GpuEngine), or, for the float64 model of the same polynomial, on arrays of
    slot values (eng None)."""

    def __init__(self, eng, target_scale: float):
        self.eng, self.s = eng, float(target_scale)

    def _chain(self, a):
        return a.chain_index() if self.eng else 0

    def to(self, a, chain):  # align_to: drop to the deeper level
        if self.eng and a.chain_index() < chain:
            return self.eng.to(a, chain)
        return a

    def align(self, a, b):  # align_pair
        c = max(self._chain(a), self._chain(b))
        return self.to(a, c), self.to(b, c)

    def lincomb(self, terms, bias: float = 0.0):
        """sum c_i a_i + bias over ciphertexts at one level and scale; the
        weights c_i are small integers (2, 1, -1) and bias a real constant."""
        if not self.eng:
            return sum(c * a for a, c in terms) + bias
        a0 = terms[0][0]
        chain = a0.chain_index()
        for a, _ in terms:
            if a.chain_index() != chain or abs(a.scale() - a0.scale()) > 1e-9 * a0.scale():
                raise ValueError("EvalMod operands differ in level or scale")
        b = int(round(bias * a0.scale())) if bias else None
        return self.eng.lincomb(terms, b, chain, a0.scale(), a0)

    def mul(self, a, b):  # multiply_and_relin, rescale_to_next, snap
        if not self.eng:
            return a * b
        r = self.eng.mul_relin_rescale(a, b)
        r.set_scale(self.s)
        return r

    def square_minus(self, a, scalar: float):  # 2 (a^2 + scalar): the reference adds, then doubles
        sq = self.mul(a, a)
        if not self.eng:
            return 2 * (sq + scalar)
        return self.eng.lincomb([(sq, 2)], 2 * int(round(scalar * sq.scale())), sq.chain_index(), sq.scale(), sq)

    def weighted_sum(self, basis, coeffs):
        """weighted_sum_chebyshev: coeffs[0] + sum_(i >= 1) coeffs[i] basis[i-1],
        the products at the basis scale squared, one rescale, snap, then the
        constant (src/evalmod.cu:266-319)."""
        terms = [(basis[i - 1], coeffs[i]) for i in range(1, len(coeffs)) if abs(coeffs[i]) >= 1e-50]
        if not terms:
            raise ValueError("weighted_sum_chebyshev: all coefficients zero")
        if not self.eng:
            acc = sum(c * t for t, c in terms)
            return acc + coeffs[0] if abs(coeffs[0]) >= 1e-50 else acc
        bs = basis[0].scale()
        chain = basis[0].chain_index()
        for t, _ in terms:
            if t.chain_index() != chain:
                raise ValueError("weighted_sum_chebyshev: basis levels differ")
        ws = [(t, int(round(c * bs))) for t, c in terms]
        acc = self.eng.rescale(self.eng.lincomb(ws, None, chain, bs * bs, basis[0]))
        acc.set_scale(self.s)
        if abs(coeffs[0]) >= 1e-50:
            acc = self.lincomb([(acc, 1)], coeffs[0])
        return acc


def _chebyshev_basis(ops: _EvalModOps, ct, max_power: int) -> list:
    """build_chebyshev_basis (src/evalmod.cu:206-264): T_1 .. T_max_power, the
    lower powers aligned to each power of two and to the last."""
    T = {1: ct}
    for n in range(2, max_power + 1):
        if n & (n - 1) == 0:
            T[n] = ops.square_minus(T[n >> 1], -0.5)
        else:
            hp2 = 1 << (n.bit_length() - 1)
            a, b = ops.align(T[hp2], T[n - hp2])
            prod = ops.lincomb([(ops.mul(a, b), 2)])
            prod, sp = ops.align(prod, T[2 * hp2 - n])
            T[n] = ops.lincomb([(prod, 1), (sp, -1)])
        if n & (n - 1) == 0 or n == max_power:
            point = n >> 1 if n & (n - 1) == 0 else 1 << (n.bit_length() - 1)
            target = ops._chain(T[n])
            for p in range(point, 0, -1):
                if p in T:
                    T[p] = ops.to(T[p], target)
    return [T[i] for i in range(1, max_power + 1)]


def _sine_k7(ops: _EvalModOps, ct):
    """sine_chebyshev_k7 (src/evalmod.cu:404-433): low + 2 T_8 high."""
    baby = _chebyshev_basis(ops, ct, 8)
    low = ops.weighted_sum(baby, _K7_LOW)
    high = ops.weighted_sum(baby[:7], _K7_HIGH)
    t8, high = ops.align(baby[7], high)
    prod = ops.lincomb([(ops.mul(t8, high), 2)])
    prod, low = ops.align(prod, low)
    return ops.lincomb([(prod, 1), (low, 1)])


def _sine_deg31(ops: _EvalModOps, ct, q_high, q_low, r_high, r_low):
    """sine_chebyshev_deg31 (src/evalmod.cu:343-402): T_16 (T_8 Q_high + Q_low)
    + T_8 R_high + R_low, the inner sums weighted_sum(T_1 .. T_7) of 8-entry
    tables (entry 0 the constant, as weighted_sum_chebyshev reads them)."""
    baby = _chebyshev_basis(ops, ct, 8)
    t16 = ops.square_minus(baby[7], -0.5)
    seven = baby[:7]
    qh, ql, rh, rl = (ops.weighted_sum(seven, c) for c in (q_high, q_low, r_high, r_low))

    def fma8(hi, lo):
        t8, hi = ops.align(baby[7], hi)
        p = ops.mul(t8, hi)
        p, lo = ops.align(p, lo)
        return ops.lincomb([(p, 1), (lo, 1)])

    Q, R = fma8(qh, ql), fma8(rh, rl)
    t16, Q = ops.align(t16, Q)
    p = ops.mul(t16, Q)
    p, R = ops.align(p, R)
    return ops.lincomb([(p, 1), (R, 1)])


def _sine_k28(ops: _EvalModOps, ct):
    """sine_chebyshev_k28 (src/evalmod.cu:464-586): baby T_1 .. T_7, giants
    T_14, T_28 and T_49 = 2 T_28 T_21 - T_7 with T_21 = 2 T_14 T_7 - T_7, then
    (ws_aux + T_28)((T_14 + Q_0) Q_1 + Q_2) + (T_14 + R_0) R_1 + R_2 - T_49."""
    baby = _chebyshev_basis(ops, ct, 7)
    t7 = baby[6]
    t14 = ops.square_minus(t7, -0.5)
    t28 = ops.square_minus(t14, -0.5)
    aux = ops.weighted_sum(baby, _K28_AUX)
    qs = [ops.weighted_sum(baby, c) for c in _K28_QUOT]
    rs = [ops.weighted_sum(baby, c) for c in _K28_REM]
    a, b = ops.align(t14, t7)
    t21 = ops.lincomb([(ops.mul(a, b), 2)])
    t21 = ops.lincomb([(t21, 1), (ops.to(t7, ops._chain(t21)), -1)])
    a, b = ops.align(t28, t21)
    t49 = ops.lincomb([(ops.mul(a, b), 2)])
    t49 = ops.lincomb([(t49, 1), (ops.to(t7, ops._chain(t49)), -1)])
    aux, t28a = ops.align(aux, t28)
    aux = ops.lincomb([(aux, 1), (t28a, 1)])

    def ps(c):
        p = ops.mul(ops.lincomb([(t14, 1), (c[0], 1)]), c[1])
        return ops.lincomb([(p, 1), (ops.to(c[2], ops._chain(p)), 1)])

    quotient, remainder = ps(qs), ps(rs)
    res = ops.mul(aux, quotient)
    res = ops.lincomb([(res, 1), (ops.to(remainder, ops._chain(res)), 1)])
    return ops.lincomb([(res, 1), (ops.to(t49, ops._chain(res)), -1)])


def _double_angle(ops: _EvalModOps, ct, R: int):
    """apply_double_angle (src/evalmod.cu:592-605): y <- 2 y^2 - (2 pi)^(-2^(j-R)),
    j = 1 .. R (the reference squares, rescales, doubles, then adds)."""
    for j in range(1, R + 1):
        scalar = -(2 * np.pi) ** (-(2.0 ** (j - R)))
        ct = ops.lincomb([(ops.mul(ct, ct), 2)], scalar)
    return ct


def _sine(ops: _EvalModOps, ct, variant: str):
    if variant == "k7_r3":
        return _sine_k7(ops, ct)
    if variant == "k16_r3":
        return _sine_deg31(ops, ct, _K16_Q_HIGH, _K16_Q_LOW, _K16_R_HIGH, _K16_R_LOW)
    if variant in ("k28_r3", "k28_r4"):
        return _sine_k28(ops, ct)
    raise ValueError(f"unknown EvalMod variant {variant!r}")


def _evalmod(context: context, ct: ciphertext, relin_keys: relin_key, variant: str) -> ciphertext:
    if ct.size() != 2 * ct._members:
        raise ValueError("EvalMod expects a size-2 ciphertext")
    need = EVALMOD_LEVELS[variant]
    if context.size_Ql(ct.chain_index()) <= need:
        raise ValueError(f"EvalMod {variant} consumes {need} levels: the ciphertext has too few primes left")
    return _evalmod_ops(_GpuEngine(context, relin_keys), ct, variant)


def _evalmod_ops(eng, ct, variant: str):
    """An EvalMod variant's operation sequence over an engine (see _GpuEngine)."""
    ops = _EvalModOps(eng, ct.scale())
    return _double_angle(ops, _sine(ops, ct, variant), EVALMOD_R[variant])


def evalmod_model(x, variant: str = "k28_r3"):
    """The polynomial an EvalMod variant evaluates, applied to the real array x
    in float64 with the same operation sequence (no encryption, no rounding
    of the constants): the value the decrypted EvalMod output approximates,
    itself an approximation of sin(2 pi K x) / (2 pi) on [-1, 1]."""
    ops = _EvalModOps(None, 1.0)
    x = np.asarray(x, dtype=np.float64)
    return _double_angle(ops, _sine(ops, x, variant), EVALMOD_R[variant])


def evalmod_k7_r3(context: context, encoder: ckks_encoder, ct: ciphertext, relin_keys: relin_key) -> ciphertext:
    """evalmod_k7_r3 (include/evalmod.h:29): degree 15, 3 double angles, 8 levels."""
    return _evalmod(context, ct, relin_keys, "k7_r3")


def evalmod_k16_r3(context: context, encoder: ckks_encoder, ct: ciphertext, relin_keys: relin_key) -> ciphertext:
    """evalmod_k16_r3 (include/evalmod.h:36): degree 31, 3 double angles, 9 levels."""
    return _evalmod(context, ct, relin_keys, "k16_r3")


def evalmod_k28_r3(context: context, encoder: ckks_encoder, ct: ciphertext, relin_keys: relin_key) -> ciphertext:
    """evalmod_k28_r3 (include/evalmod.h:45): degree 49, 3 double angles, 9 levels."""
    return _evalmod(context, ct, relin_keys, "k28_r3")


def evalmod_k28_r4(context: context, encoder: ckks_encoder, ct: ciphertext, relin_keys: relin_key) -> ciphertext:
    """evalmod_k28_r4 (include/evalmod.h:55): the K = 28 polynomial with a fourth
    double angle, 10 levels.  As in the reference, the polynomial is tuned for
    three steps, so the result is not sin(2 pi 28 x) / (2 pi) (the reference's
    own test leaves this variant disabled, test/evalmod_test.cu:236-243)."""
    return _evalmod(context, ct, relin_keys, "k28_r4")


def _times_i(ctx, ct: ciphertext, sign: int = 1) -> ciphertext:
    """ct * (sign i): the plaintext polynomial times sign X^(N/2), exact."""
    L = ctx.size_Ql(ct.chain_index())

    def make():
        c = np.zeros(ctx.N, dtype=np.int64)
        c[ctx.N // 2] = sign
        return ctx._ntt(ctx._signed_to_rns(c, L), L)

    mono = ctx._cached_const(("times_i", sign, L), make)
    out = ctx._empty(*ct.data.shape)
    ctx.native.ct_multiply_plain(ct.data, mono, out, L)
    return ct._like(out)


def _times_int(ctx, ct: ciphertext, k: int) -> ciphertext:
    """ct times the integer k (|k| < 2^63), residue by residue; scale unchanged
    (the reference's multiply_uint_scalars_per_tower)."""
    L = ctx.size_Ql(ct.chain_index())
    out = ctx._empty(*ct.data.shape)
    _ct_lincomb(ctx, L, [ct.data], [int(k)], out, None, ct._members)
    return ct._like(out)


def _scale_up_for_bootstrap(ctx, ct: ciphertext, current_scale: float) -> ciphertext:
    """scale_up_for_bootstrap (src/bootstrap.cu:1435-1510): a ciphertext one
    level above the bottom ([q_msg, q_scale]; fresher ones are switched down
    first) times c0 = round(q_msg q_scale / current_scale), rescaled: scale
    q_msg at the bottom.  At the bottom already: nothing if the scale is q_msg,
    else times round(q_msg / current_scale)."""
    from fractions import Fraction

    bottom = ctx.size_Q
    q_msg = ctx.moduli[0]
    cs = Fraction(current_scale)
    if ct.chain_index() == bottom:
        if abs(current_scale / q_msg - 1.0) < 1e-6:
            ct.set_scale(float(q_msg))
            return ct
        c0 = round(Fraction(q_msg) / cs)
        if c0 == 0:
            raise ValueError("scale_up_for_bootstrap: at bottom but ratio q_msg/current_scale rounds to 0")
        out = _times_int(ctx, ct, c0)
        out.set_scale(current_scale * c0)
        return out
    if ct.chain_index() < bottom - 1:
        ct = mod_switch_to(ctx, ct, bottom - 1)
    c0 = round(Fraction(q_msg * ctx.moduli[1]) / cs)
    if not 0 < c0 < (1 << 63):
        raise ValueError("scale_up_for_bootstrap: scale ratio out of range")
    out = _times_int(ctx, ct, c0)
    out.set_scale(current_scale * c0)
    out = rescale_to_next(ctx, out)
    out.set_scale(float(q_msg))
    return out


def _eval_round(ctx, ct: ciphertext, rk: relin_key) -> ciphertext:
    """eval_round_k28_r3 (src/bootstrap.cu:1661-1680): K ct - evalmod_k28_r3(ct),
    ~ the integer part, K = 28."""
    kct = _times_int(ctx, ct, 28)
    em = _evalmod(ctx, ct, rk, "k28_r3")
    kct = mod_switch_to(ctx, kct, em.chain_index())
    kct.set_scale(em.scale())
    return sub(ctx, kct, em)


def _bootstrap_evalround(ctx, ct: ciphertext, bk: bootstrap_key, user_scale: float,
                         split_scale_down: bool) -> ciphertext:
    """The reference's bootstrap (src/bootstrap.cu:1703-1951) on this build's
    transforms: scale-up to q_msg, ModRaise (saved), CoeffToSlot, conjugate
    split, EvalRound on both tracks, recombination, SlotToCoeff (the rounding
    part qi), then saved brought to qi's level and exact scale by one integer
    multiply and rescale, minus qi; with split_scale_down the small result is
    then brought to user_scale by one more integer multiply and rescale."""
    from fractions import Fraction

    if bk.eval_mod_levels < EVALMOD_LEVELS["k28_r3"]:
        raise RuntimeError("bootstrap: ct deeper than S2C start — eval_mod_levels mismatch")
    if split_scale_down != bk.split_scale_down:
        raise ValueError("split_scale_down differs from the bootstrap key's")
    if user_scale <= 0.0:
        raise ValueError("user_scale must be > 0")
    q_msg = ctx.moduli[0]
    ct = _scale_up_for_bootstrap(ctx, ct, user_scale)
    saved = mod_raise_inplace(ctx, ct, bk.small)
    saved.set_scale(float(q_msg))
    # CoeffToSlot; its last rescale waits until the conjugate split is done
    u = _transform(ctx, saved, bk.c2s, bk.c2s_pts, bk.glk, bk.c2s_boost, last_rescale=False)
    conj = apply_galois(ctx, u, 2 * ctx.N - 1, bk.glk)
    real = rescale_to_next(ctx, add(ctx, u, conj))
    imag = rescale_to_next(ctx, _times_i(ctx, sub(ctx, u, conj), -1))
    # both tracks through EvalRound in lockstep: one batched call per step
    real, imag = _unbundle(_eval_round(ctx, _bundle(ctx, [real, imag]), bk.rlk))
    imag = _times_i(ctx, imag, 1)
    c = max(real.chain_index(), imag.chain_index())
    real, imag = mod_switch_to(ctx, real, c), mod_switch_to(ctx, imag, c)
    imag.set_scale(real.scale())
    out = add(ctx, real, imag)
    if out.chain_index() > bk.s2c_start:
        raise RuntimeError("bootstrap: ct deeper than S2C start — eval_mod_levels mismatch")
    out = mod_switch_to(ctx, out, bk.s2c_start)
    out.set_scale(float(ctx.moduli[ctx.size_Ql(bk.s2c_start) - 1]))
    out = _transform(ctx, out, bk.s2c, bk.s2c_pts, bk.glk, bk.s2c_boost)
    qi_chain = out.chain_index()
    if abs(out.scale() - saved.scale()) > 0.5:
        saved = mod_switch_to(ctx, saved, qi_chain - 1)
        q_back = ctx.moduli[ctx.size_Ql(qi_chain - 1) - 1]
        D = round(Fraction(out.scale()) * q_back / q_msg)
        if not 0 < D < (1 << 63):
            raise ValueError("bootstrap: scale alignment factor out of range")
        saved = _times_int(ctx, saved, D)
        saved.set_scale(saved.scale() * D)
        saved = rescale_to_next(ctx, saved)
    saved = mod_switch_to(ctx, saved, qi_chain)
    saved.set_scale(out.scale())
    res = sub(ctx, saved, out)
    if split_scale_down:
        q_drop = ctx.moduli[ctx.size_Ql(qi_chain) - 1]
        D2 = round(Fraction(q_drop) * Fraction(user_scale) / Fraction(res.scale()))
        if not 0 < D2 < (1 << 63):
            raise ValueError("bootstrap: scale-down factor out of range")
        res = _times_int(ctx, res, D2)
        res.set_scale(res.scale() * D2)
        res = rescale_to_next(ctx, res)
        res.set_scale(float(user_scale))
    return res


def bootstrap(context: context, encoder: ckks_encoder, ct: ciphertext, bk: bootstrap_key, user_scale: float,
              split_scale_down: bool = False) -> ciphertext:
    """bootstrap (src/bootstrap.cu:1703-1951, python/src/binding.cu:329-336).

    With a "k28_r3" key: the reference's pipeline (_bootstrap_evalround); the
    result is at chain 4 + eval_mod_levels + 3 (one more with
    split_scale_down) at scale user_scale (the key's baked SlotToCoeff scale,
    or the split's last step).  split_scale_down must match the key's.

    With a "cheb63" key: a ciphertext at scale user_scale, at any level (it is
    brought to the bottom of the chain first) -> the same message at chain
    index 1 + 2 * (transform layers) + 10, at a scale within a few parts in
    10^12 of user_scale (the exact value is carried); split_scale_down must be
    false."""
    if ct.size() != 2:
        raise ValueError("bootstrap expects a size-2 ciphertext")
    if bk.evalmod == "k28_r3":
        return _bootstrap_evalround(context, ct, bk, user_scale, split_scale_down)
    ctx = context
    if split_scale_down:
        raise ValueError("split_scale_down applies to the 'k28_r3' pipeline only")
    if abs(ct.scale() - user_scale) > 1e-6 * user_scale:
        raise ValueError("ciphertext scale differs from user_scale")
    q0 = ctx.moduli[0]
    ct = mod_switch_to(ctx, ct, ctx.size_Q)
    # exact integer lift of the message to ~q0 / 2^BOOT_MSG_BITS: EvalMod's
    # sin(2 pi x) / (2 pi) ~ x then holds to (2 pi 2^-12)^2 / 6 ~ 4e-7 relative,
    # and the noise that the transforms add is magnified q0 / scale times less
    k = max(0, int(np.floor(np.log2(q0 / user_scale))) - BOOT_MSG_BITS)
    scale = float(user_scale)
    if k:
        ct = multiply_plain(ctx, ct, _const_plain(ctx, 1 << k, 1.0, ctx.size_Q))
        scale *= 2.0 ** k
    raised = mod_raise_inplace(ctx, ct, bk.small)
    raised.set_scale(float(q0))  # slots now read coefficients / q0 = I + m scale / q0
    # CoeffToSlot; its last rescale waits until the conjugate split is done,
    # so the conjugation's key-switching noise lands at the larger scale too
    u = _transform(ctx, raised, bk.c2s, bk.c2s_pts, bk.glk, bk.c2s_boost, last_rescale=False)
    conj = apply_galois(ctx, u, 2 * ctx.N - 1, bk.glk)
    real = rescale_to_next(ctx, add(ctx, u, conj))                     # Re(x) / K
    imag = rescale_to_next(ctx, _times_i(ctx, sub(ctx, u, conj), -1))  # Im(x) / K
    # both tracks through EvalMod in lockstep: one batched call per step
    real, imag = _unbundle(_eval_mod(ctx, _bundle(ctx, [real, imag]), bk))
    y = add(ctx, real, _times_i(ctx, imag, 1))
    out = apply_s2c_inplace(ctx, y, bk)
    out.set_scale(scale * out.scale() / q0)
    return out


# ---------------------------------------------------------------- CKKS engine
class ckks_engine_config:
    """CKKSEngineConfig (include/ckks_engine.h:29-95, python/src/binding.cu:339-355):
    the knobs of the bootstrappable facade, with the reference's defaults."""

    def __init__(self):
        self.log_n = 16
        self.user_scale = 2.0 ** 40
        self.num_scale_levels = 14
        self.sparse_hw = 128
        self.num_special_primes = 6
        self.include_user_rotations = True
        self.user_rotation_steps = []
        self.user_rotation_target_chain_indices = []
        self.split_scale_down = False
        self.build_two_scale_arrays = False
        self.use_bootstrap_to_17_levels = False


def _long_double(v: int):
    """The integer 0 <= v < 2^64 as a numpy long double, exactly (the x87
    extended format of x86-64 has a 64-bit significand), as the reference's
    static_cast<long double>(uint64_t) makes it."""
    return np.longdouble(v >> 32) * np.longdouble(1 << 32) + np.longdouble(v & 0xFFFFFFFF)


# EvalMod levels of the engine's pipeline (evalmod_k28_r3: 6 sine + 3 double angle)
_ENGINE_EVALMOD_LEVELS = 9


class ckks_engine:
    """CKKSEngine (src/ckks_engine.cu, include/ckks_engine.h) with the methods
    its Python binding exposes (python/src/binding.cu:357-382): a CKKS context
    on a bootstrappable chain, its secret, relinearization, bootstrap and user
    rotation keys, where the caller sees a user_level counter only.  User level
    0 is the freshest level of the user-scale segment, each rescale adds 1,
    max_user_level() = num_scale_levels - 1 is the deepest one (two primes
    left), and bootstrap_inplace brings a ciphertext at any user level back to
    user level 0 (1 with split_scale_down).

    Chain (src/ckks_engine.cu:76-127), bottom to top, then the special primes:
      default:  58 | 40 x num_scale_levels | 58 x 3 | 58 x 9 | 29 x 3 | 58 x special
      use_bootstrap_to_17_levels: 40 x num_scale_levels | 29 | 54 x 12 | 42 | 60 x special
    (the second chain only: encode / encrypt / decrypt; bootstrap_inplace
    refuses it, as the reference does).  Residues follow the library's
    bootstrap and key switching; the keys come from this build's seedable
    sampler (`seed`), so they equal the reference's only given the same key
    material."""

    def __init__(self, config: ckks_engine_config | None = None, seed=None):
        import copy

        cfg = copy.deepcopy(config) if config is not None else ckks_engine_config()
        self._cfg = cfg
        if int(cfg.log_n) != 16:
            raise ValueError("CKKSEngine: this port pins log_n=16")
        nsl, nsp = int(cfg.num_scale_levels), int(cfg.num_special_primes)
        if nsl < 2:
            raise ValueError("CKKSEngine: num_scale_levels must be >= 2")
        if nsp < 1:
            raise ValueError("CKKSEngine: num_special_primes must be >= 1")
        size_Q = nsl + 14 if cfg.use_bootstrap_to_17_levels else 1 + nsl + 3 + 9 + 3
        if size_Q % nsp:
            raise ValueError("CKKSEngine: size_Q must be divisible by num_special_primes "
                             "(required by the hybrid KSK decomposition).")
        N = 1 << int(cfg.log_n)
        if cfg.use_bootstrap_to_17_levels:
            bits = [40] * nsl + [29] + [54] * 12 + [42] + [60] * nsp
        else:
            bits = ckks_engine_coeff_bits(nsl, nsp)
        # Galois elements: the CoeffToSlot / SlotToCoeff steps, the user steps
        # (the explicit list, else +-1 and +-2), then conjugation
        stages = [5, 5, 5]
        c2s, s2c = build_c2s_diagonals(cfg.log_n, stages), build_s2c_diagonals(cfg.log_n, stages)
        boot_steps = set(c2s_required_rotation_steps(c2s, N // 2)) | set(c2s_required_rotation_steps(s2c, N // 2))
        if cfg.user_rotation_steps:
            user_steps = [int(s) for s in cfg.user_rotation_steps]
        elif cfg.include_user_rotations:
            user_steps = [1, -1, 2, -2]
        else:
            user_steps = []
        conj = 2 * N - 1
        elts = get_elts_from_steps(sorted(boot_steps | set(user_steps)), N) + [conj]
        p = params(scheme_type.ckks)
        p.set_poly_modulus_degree(N)
        p.set_special_modulus_size(nsp)
        p.set_coeff_modulus(create_coeff_modulus(N, bits))
        p.set_galois_elts(elts)
        self._ctx = context(p)
        rng = _rng(seed)
        self._sk = secret_key(self._ctx, seed=rng)
        self._enc = ckks_encoder(self._ctx)
        self._bk = None
        self._user_glk = galois_key(self._ctx.galois_elts)
        first = self._ctx.get_first_index()
        self._bottom = self._ctx.total_parm_size() - 1
        self._ckks_scale, self._ckks_rescaled_scale = [], []
        if cfg.use_bootstrap_to_17_levels:
            # CoeffToSlot 1 + EvalRound 9 + SlotToCoeff 3 primes above the
            # user segment, whose first rescale drops the 29-bit prime
            self._freshest = first + 13
            if self._freshest + nsl != self._bottom:
                raise RuntimeError("CKKSEngine: BootstrapTo17Levels chain mismatch: "
                                   "freshest + num_scale_levels != bottom.")
            if cfg.build_two_scale_arrays:
                self._build_scale_arrays()
            return
        self._bk = create_bootstrap_key(self._ctx, self._enc, self._sk, sparse_hamming_weight=int(cfg.sparse_hw),
                                        eval_mod_levels=_ENGINE_EVALMOD_LEVELS, user_scale=float(cfg.user_scale),
                                        split_scale_down=bool(cfg.split_scale_down), stages_per_layer=stages,
                                        seed=rng)
        nl = len(stages)
        self._freshest = first + nl + _ENGINE_EVALMOD_LEVELS + nl
        if self._freshest + nsl != self._bottom:
            raise RuntimeError("CKKSEngine: chain layout mismatch: freshest + num_scale_levels != bottom. "
                               "Check chain construction.")
        glk = self._bk.glk
        if not user_steps:
            # the bootstrap key's user bundle: conjugation only
            self._user_glk.keys[conj] = glk.keys[conj]
        else:
            targets = [int(t) for t in cfg.user_rotation_target_chain_indices]
            if targets:
                if not cfg.user_rotation_steps:
                    raise ValueError("CKKSEngine: user_rotation_target_chain_indices set but "
                                     "user_rotation_steps is empty")
                if len(targets) != len(cfg.user_rotation_steps):
                    raise ValueError("CKKSEngine: user_rotation_target_chain_indices size "
                                     "must match user_rotation_steps size")
            index = {e: i for i, e in enumerate(self._ctx.galois_elts)}

            def find_idx(elt):
                if elt not in index:
                    raise RuntimeError("CKKSEngine: configured galois elt not in registered set")
                return index[elt]

            # conjugation with the partitions of the one level the bootstrap
            # applies it at (here before CoeffToSlot's last rescale, chain
            # first + nl - 1; the reference's pipeline rescales first and uses
            # first + nl); a user step that CoeffToSlot / SlotToCoeff also use
            # shares that key instead of getting one of its own
            # (src/ckks_engine.cu:227-379)
            idxs, levels, shared = [find_idx(conj)], [first + nl - 1], []
            for i, step in enumerate(user_steps):
                elt = get_elt_from_step(step, N)
                j = find_idx(elt)
                if step in boot_steps:
                    shared.append(elt)
                    continue
                idxs.append(j)
                levels.append(targets[i] if targets else self._freshest)
            self._user_glk = self._sk.create_galois_keys_per_level(self._ctx, idxs, levels, seed=rng)
            for elt in shared:
                self._user_glk.keys[elt] = glk.keys[elt]
            # the bootstrap's conjugation reads the user bundle's key
            glk.keys[conj] = self._user_glk.keys[conj]
        if cfg.build_two_scale_arrays:
            self._build_scale_arrays()

    def _build_scale_arrays(self):
        """build_scale_arrays (src/ckks_engine.cu:435-460) in long double:
        ckks_scale[i] = the squared scale at chain index i, starting from
        user_scale^2; ckks_rescaled_scale[i] = ckks_scale[i] / (that level's last
        prime), and ckks_scale[i + 1] = ckks_rescaled_scale[i]^2."""
        ctx = self._ctx
        cur = np.longdouble(float(self._cfg.user_scale)) ** 2
        sc, rs = [], []
        for idx in range(ctx.total_parm_size()):
            sc.append(cur)
            last = ctx.moduli[-1] if idx == 0 else ctx.moduli[ctx.size_Ql(idx) - 1]
            r = cur / _long_double(last)
            rs.append(r)
            cur = r * r
        self._ckks_scale, self._ckks_rescaled_scale = sc, rs

    # ---- user-facing properties
    def slot_count(self) -> int:
        return self._ctx.N // 2

    def user_scale(self) -> float:
        return float(self._cfg.user_scale)

    def max_user_level(self) -> int:
        return int(self._cfg.num_scale_levels) - 1

    def user_level(self, ct: ciphertext) -> int:
        ci = ct.chain_index()
        if ci < self._freshest or ci > self._bottom - 1:
            raise ValueError("CKKSEngine::user_level: ciphertext chain_index is outside the user-scale segment")
        return ci - self._freshest

    def user_level_chain_index(self, user_level: int) -> int:
        if user_level < 0 or user_level >= int(self._cfg.num_scale_levels):
            raise ValueError("CKKSEngine::user_level_chain_index: user_level out of range")
        return self._freshest + int(user_level)

    # ---- encoding / encryption
    def encode(self, values, user_level: int = 0) -> plaintext:
        """CKKSEngine::encode (src/ckks_engine.cu:487-499): complex slot values
        at user_scale, at the user level's chain index."""
        if user_level < 0 or user_level >= int(self._cfg.num_scale_levels):
            raise ValueError("CKKSEngine::encode: user_level out of range")
        return self._enc.encode_complex_vector(self._ctx, values, float(self._cfg.user_scale),
                                               self._freshest + int(user_level))

    def encrypt(self, pt: plaintext, seed=None) -> ciphertext:
        return self._sk.encrypt_symmetric(self._ctx, pt, seed=seed)

    def decrypt_decode(self, ct: ciphertext) -> list:
        return self._enc.decode_complex_vector(self._ctx, self._sk.decrypt(self._ctx, ct))

    # ---- arithmetic and level management (the C++ class's, src/ckks_engine.cu:515-551)
    @staticmethod
    def _set(dst: ciphertext, r: ciphertext) -> None:
        dst.__dict__.update(r.__dict__)  # data, level, scale and the rest of the state

    def add_inplace(self, dst: ciphertext, src: ciphertext) -> None:
        self._set(dst, add(self._ctx, dst, src))

    def sub_inplace(self, dst: ciphertext, src: ciphertext) -> None:
        self._set(dst, sub(self._ctx, dst, src))

    def mul_and_relin_inplace(self, dst: ciphertext, src: ciphertext) -> None:
        self._set(dst, multiply_and_relin(self._ctx, dst, src, self.relin_key()))

    def mul_plain_inplace(self, dst: ciphertext, pt: plaintext) -> None:
        self._set(dst, multiply_plain(self._ctx, dst, pt))

    def rescale_inplace(self, ct: ciphertext) -> None:
        """rescale_to_next, refused from the deepest user level (the next
        level, one prime, is the bootstrap's own)."""
        if ct.chain_index() >= self._bottom - 1:
            raise RuntimeError("CKKSEngine::rescale_inplace: ciphertext is already at max user_level "
                               "(pre_boot_index); call bootstrap_inplace next.")
        self._set(ct, rescale_to_next(self._ctx, ct))

    def rotate_inplace(self, ct: ciphertext, step: int) -> None:
        self._set(ct, rotate(self._ctx, ct, step, self._user_glk))

    # ---- bootstrap
    def bootstrap_inplace(self, ct: ciphertext) -> None:
        """CKKSEngine::bootstrap_inplace (src/ckks_engine.cu:553-601): a
        ciphertext at any user level is switched down to the deepest one,
        its scale set to user_scale, bootstrapped, and lands at user level 0
        (1 with split_scale_down) at scale user_scale."""
        if self._cfg.use_bootstrap_to_17_levels:
            raise RuntimeError("CKKSEngine::bootstrap_inplace: use_bootstrap_to_17_levels chain does not have "
                               "a bootstrap algorithm yet.")
        self.user_level(ct)
        pre_boot = self._bottom - 1
        if ct.chain_index() != pre_boot:
            mod_switch_to_inplace(self._ctx, ct, pre_boot)
        ct.set_scale(float(self._cfg.user_scale))
        out = bootstrap(self._ctx, self._enc, ct, self._bk, float(self._cfg.user_scale),
                        bool(self._cfg.split_scale_down))
        expected = self._freshest + (1 if self._cfg.split_scale_down else 0)
        if out.chain_index() != expected:
            raise RuntimeError("CKKSEngine::bootstrap_inplace: post-bootstrap chain_index != expected")
        self._set(ct, out)
        ct.set_scale(float(self._cfg.user_scale))

    # ---- read-only views
    def context(self) -> context:
        return self._ctx

    def encoder(self) -> ckks_encoder:
        return self._enc

    def secret_key(self) -> secret_key:
        return self._sk

    def relin_key(self) -> relin_key:
        return self._bk.rlk if self._bk is not None else relin_key()

    def galois_key(self) -> galois_key:
        return self._user_glk

    def bootstrap_key(self) -> bootstrap_key:
        return self._bk

    # ---- per-level scale arrays (build_two_scale_arrays)
    def scale_array_size(self) -> int:
        return len(self._ckks_rescaled_scale)

    def ckks_scale_at(self, chain_index: int) -> float:
        return float(self._ckks_scale[chain_index]) if chain_index < len(self._ckks_scale) else 0.0

    def ckks_rescaled_scale_at(self, chain_index: int) -> float:
        return (float(self._ckks_rescaled_scale[chain_index])
                if chain_index < len(self._ckks_rescaled_scale) else 0.0)


# ---------------------------------------------------------------- slot sums, polynomials
def inner_sum(context: context, galois_key: galois_key, ct: ciphertext, block_size: int) -> ciphertext:
    """inner_sum (src/linear.cu:9-25): each block_size-wide block's sum in its
    first slot (the other slots hold partial sums), by log2(block_size)
    rotate-and-add steps with strides 1, 2, 4, ..."""
    block_size = int(block_size)
    if block_size == 0 or block_size & (block_size - 1):
        raise ValueError("inner_sum: block_size must be a power of 2")
    acc, stride = ct, 1
    while stride < block_size:
        acc = add(context, acc, rotate(context, acc, stride, galois_key))
        stride <<= 1
    return acc


def replicate(context: context, galois_key: galois_key, ct: ciphertext, period: int, num_slots: int) -> ciphertext:
    """replicate (src/linear.cu:27-50): slots [0, period) copied into every
    period of num_slots (slot k period + i = slot i, given the other slots
    start at zero), by rotations by -period, -2 period, ... and additions."""
    period, num_slots = int(period), int(num_slots)
    if period == 0 or period & (period - 1):
        raise ValueError("replicate: period must be a power of 2")
    if num_slots == 0 or num_slots & (num_slots - 1):
        raise ValueError("replicate: num_slots must be a power of 2")
    if period > num_slots:
        raise ValueError("replicate: period exceeds num_slots")
    acc, stride = ct, period
    while stride < num_slots:
        acc = add(context, acc, rotate(context, acc, -stride, galois_key))
        stride <<= 1
    return acc


def _ps_mul_scalar(ctx: context, ct: ciphertext, c: float, nominal: float) -> ciphertext:
    """ct * c by a constant plaintext at the scale of the level's last prime,
    a rescale, and the scale set back to `nominal` (src/ps.cu:26-39)."""
    q = float(ctx.moduli[ctx.size_Ql(ct.chain_index()) - 1])
    out = rescale_to_next(ctx, multiply_plain(ctx, ct, _const_plain(ctx, c, q, ct.chain_index())))
    out.set_scale(nominal)
    return out


def _ps_add_scalar(ctx: context, ct: ciphertext, c: float) -> ciphertext:
    """ct + c in ceil(|c| / 100) equal pieces, each encoded at the ciphertext's
    scale (src/ps.cu:52-66)."""
    if c == 0.0:
        return ct
    pieces = max(1, int(np.ceil(abs(c) / 100.0)))
    piece = c / pieces
    for _ in range(pieces):
        ct = add_plain(ctx, ct, _const_plain(ctx, piece, ct.scale(), ct.chain_index()))
    return ct


def _ps_chunk(ctx, coeffs, babies, k: int, m: int, target: int, nominal: float) -> ciphertext:
    """c_k(x) = a_(k m) + sum_(j = 1 .. m-1) a_(k m + j) x^j at chain index
    `target` (src/ps.cu:72-124): each nonzero linear term is its baby switched
    to target - 1 and multiplied by the scalar (which brings it to target)."""
    d, base = len(coeffs) - 1, k * m
    terms = [(j, coeffs[base + j]) for j in range(1, m) if base + j <= d and coeffs[base + j] != 0.0]
    const = coeffs[base] if base <= d else 0.0
    prev = target - 1 if target > 0 else 0
    acc = None
    for j, a in terms or [(1, 0.0)]:  # no linear term: a zero at target via x * 0
        t = mod_switch_to(ctx, babies[j - 1], prev)
        t = _ps_mul_scalar(ctx, t, a, nominal)
        acc = t if acc is None else add(ctx, acc, t)
    return _ps_add_scalar(ctx, acc, const)


def eval_polynomial(context: context, encoder: ckks_encoder, relin_key: relin_key, ct: ciphertext,
                    coeffs) -> ciphertext:
    """eval_polynomial (src/ps.cu:129-200, include/ps.h): p(x) = a_0 + a_1 x +
    ... + a_d x^d by Paterson-Stockmeyer with m = ceil(sqrt(d + 1)) baby powers
    and l = ceil((d + 1) / m) giant chunks in Horner order; every product is
    rescaled and its scale set back to the input's.  The result is at chain
    index ct.chain_index() + m + l - 2 (include/ps.h states m + l - 1; its
    code, followed here step for step, consumes one level less).  Constants
    are encoded exactly (coefficient 0 = round(c scale))."""
    ctx = context
    coeffs = [float(c) for c in coeffs]
    if len(coeffs) < 2:
        raise ValueError("eval_polynomial: degree must be >= 1")
    d = len(coeffs) - 1
    m = int(np.ceil(np.sqrt(d + 1.0)))
    l = (d + 1 + m - 1) // m
    nominal, c0 = ct.scale(), ct.chain_index()
    # baby powers x^1 .. x^(m-1)
    babies, x_run = [ct], ct
    for i in range(2, m):
        nxt = rescale_to_next(ctx, multiply_and_relin(ctx, babies[i - 2], x_run, relin_key))
        nxt.set_scale(nominal)
        babies.append(nxt)
        if i < m - 1:  # x_run one level down, to meet babies[i - 1]
            x_run = _ps_mul_scalar(ctx, x_run, 1.0, nominal)
    baby_lvl = c0 + m - 2 if m >= 2 else c0
    babies = [mod_switch_to(ctx, b, baby_lvl) for b in babies]
    x_run = mod_switch_to(ctx, x_run, baby_lvl)
    # giant base x^m
    x_m = None
    if l >= 2:
        x_m = rescale_to_next(ctx, multiply_and_relin(ctx, babies[-1], x_run, relin_key))
        x_m.set_scale(nominal)
    # Horner over the giant chunks
    result = _ps_chunk(ctx, coeffs, babies, l - 1, m, baby_lvl + 1, nominal)
    for kk in range(l - 2, -1, -1):
        if x_m is None:
            raise RuntimeError("eval_polynomial: x_m absent with l>=2")
        x_m = mod_switch_to(ctx, x_m, result.chain_index())
        result = rescale_to_next(ctx, multiply_and_relin(ctx, result, x_m, relin_key))
        result.set_scale(nominal)
        result = add(ctx, result, _ps_chunk(ctx, coeffs, babies, kk, m, result.chain_index(), nominal))
    return result
