"""ctypes view of the C oracle (oracle/ckks_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py as the checker / CPU baseline.  The product path
(phantom-fhe_amd/) never imports this module.

All arrays are numpy uint64, C-contiguous, limb-major ([..., L, N]).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_ckks.so")

_u64p = C.POINTER(C.c_uint64)
_u32p = C.POINTER(C.c_uint32)


def _load():
    if not os.path.exists(_LIB_PATH):
        raise RuntimeError(f"oracle library not built: {_LIB_PATH} (run `make -C oracle`)")
    lib = C.CDLL(_LIB_PATH)
    sz, u64, vp, i32 = C.c_size_t, C.c_uint64, C.c_void_p, C.c_int
    sig = {
        "orc_is_prime": (i32, [u64]),
        "orc_create_coeff_modulus": (i32, [u64, C.POINTER(C.c_int), sz, _u64p]),
        "orc_minimal_primitive_root": (u64, [u64, u64]),
        "orc_mulmod": (u64, [u64, u64, u64]),
        "orc_powmod": (u64, [u64, u64, u64]),
        "orc_invmod": (u64, [u64, u64]),
        "orc_shoup": (u64, [u64, u64]),
        "orc_ntt_tables": (None, [u64, u64, _u64p, _u64p, _u64p, _u64p, _u64p, _u64p]),
        "orc_ntt_fwd_limb": (None, [_u64p, u64, u64, _u64p, _u64p]),
        "orc_ntt_inv_limb": (None, [_u64p, u64, u64, _u64p, _u64p, u64]),
        "orc_ntt_naive_limb": (None, [_u64p, _u64p, u64, u64, u64]),
        "orc_ctx_create": (vp, [u64, _u64p, sz, sz]),
        "orc_ctx_destroy": (None, [vp]),
        "orc_ctx_table": (_u64p, [vp, sz, i32]),
        "orc_ctx_root": (u64, [vp, sz]),
        "orc_ntt_fwd": (None, [vp, _u64p, sz, sz, sz, i32]),
        "orc_ntt_inv": (None, [vp, _u64p, sz, sz, sz, i32]),
        "orc_tensor": (None, [vp, sz, _u64p, _u64p, _u64p]),
        "orc_beta": (sz, [vp, sz]),
        "orc_dnum": (sz, [vp]),
        "orc_modup": (None, [vp, sz, _u64p, _u64p, i32]),
        "orc_ks_inner_prod": (None, [vp, sz, _u64p, _u64p, sz, _u64p]),
        "orc_moddown": (None, [vp, sz, _u64p, _u64p, i32]),
        "orc_keyswitch": (i32, [vp, sz, _u64p, _u64p, _u64p, sz, i32]),
        "orc_multiply_and_relin": (i32, [vp, sz, _u64p, _u64p, _u64p, sz, _u64p, i32]),
        "orc_rescale": (None, [vp, sz, _u64p, sz, _u64p, i32]),
        "orc_elt_from_step": (C.c_uint32, [i32, u64]),
        "orc_galois_perm": (None, [u64, C.c_uint32, _u32p]),
        "orc_apply_galois_ntt": (None, [u64, C.c_uint32, _u64p, _u64p, sz]),
        "orc_apply_galois": (i32, [vp, sz, _u64p, C.c_uint32, _u64p, sz, i32]),
        "orc_hoist_rotations": (i32, [vp, sz, _u64p, _u32p, sz, C.POINTER(_u64p), sz, _u64p, i32]),
        "orc_hoisting": (i32, [vp, sz, _u64p, _u32p, sz, C.POINTER(_u64p), sz, _u64p, i32]),
        "orc_kswitch_key": (None, [vp, _u64p, _u64p, _u64p, _u64p, _u64p]),
        "orc_mul_poly": (None, [vp, sz, sz, _u64p, _u64p, _u64p]),
        "orc_build_info": (C.c_char_p, []),
    }
    for name, (res, args) in sig.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def _p(a: np.ndarray):
    assert a.dtype == np.uint64 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data_as(_u64p)


def u64(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint64))


def build_info() -> str:
    """Compiler and flags the oracle library was built with."""
    return lib().orc_build_info().decode()


def threads_default() -> int:
    return int(os.environ.get("ORACLE_THREADS", "1"))


# ---------------------------------------------------------------- scalars
def is_prime(n: int) -> bool:
    return bool(lib().orc_is_prime(n))


def create_coeff_modulus(N: int, bit_sizes) -> list[int]:
    bits = (C.c_int * len(bit_sizes))(*bit_sizes)
    out = np.zeros(len(bit_sizes), dtype=np.uint64)
    if lib().orc_create_coeff_modulus(N, bits, len(bit_sizes), _p(out)) != 0:
        raise ValueError("failed to find enough qualifying primes")
    return [int(x) for x in out]


def minimal_primitive_root(degree: int, q: int) -> int:
    return int(lib().orc_minimal_primitive_root(degree, q))


def ntt_tables(N: int, q: int):
    tw, tws, itw, itws = (np.zeros(N, dtype=np.uint64) for _ in range(4))
    ni, nis = C.c_uint64(0), C.c_uint64(0)
    lib().orc_ntt_tables(N, q, _p(tw), _p(tws), _p(itw), _p(itws), C.byref(ni), C.byref(nis))
    return tw, tws, itw, itws, int(ni.value), int(nis.value)


def ntt_naive(a: np.ndarray, q: int, psi: int) -> np.ndarray:
    a = u64(a)
    out = np.zeros_like(a)
    lib().orc_ntt_naive_limb(_p(a), _p(out), a.shape[-1], q, psi)
    return out


def elt_from_step(step: int, N: int) -> int:
    return int(lib().orc_elt_from_step(step, N))


def galois_perm(N: int, elt: int) -> np.ndarray:
    perm = np.zeros(N, dtype=np.uint32)
    lib().orc_galois_perm(N, elt, perm.ctypes.data_as(_u32p))
    return perm


# ---------------------------------------------------------------- context
class Oracle:
    """Key-level context over all |QP| primes (Q primes then P primes)."""

    def __init__(self, N: int, moduli, size_P: int):
        self.N = N
        self.moduli = [int(m) for m in moduli]
        self.size_QP = len(self.moduli)
        self.size_P = size_P
        self.size_Q = self.size_QP - size_P
        m = u64(self.moduli)
        self._ctx = lib().orc_ctx_create(N, _p(m), self.size_QP, size_P)

    def __del__(self):
        if getattr(self, "_ctx", None):
            lib().orc_ctx_destroy(self._ctx)
            self._ctx = None

    # chain helpers
    def size_Ql(self, chain_index: int) -> int:
        return self.size_Q - (chain_index - 1)

    def beta(self, chain_index: int) -> int:
        return int(lib().orc_beta(self._ctx, chain_index))

    @property
    def dnum(self) -> int:
        return int(lib().orc_dnum(self._ctx))

    def table(self, idx: int, which: int) -> np.ndarray:
        n = 1 if which >= 4 else self.N
        ptr = lib().orc_ctx_table(self._ctx, idx, which)
        return np.ctypeslib.as_array(ptr, shape=(n,)).copy()

    def root(self, idx: int) -> int:
        return int(lib().orc_ctx_root(self._ctx, idx))

    # transforms
    def ntt_fwd(self, data: np.ndarray, start: int = 0, threads: int | None = None) -> np.ndarray:
        d = u64(data).copy()
        L = d.shape[-2]
        M = d.size // (L * self.N)
        lib().orc_ntt_fwd(self._ctx, _p(d), M, L, start, threads or threads_default())
        return d

    def ntt_inv(self, data: np.ndarray, start: int = 0, threads: int | None = None) -> np.ndarray:
        d = u64(data).copy()
        L = d.shape[-2]
        M = d.size // (L * self.N)
        lib().orc_ntt_inv(self._ctx, _p(d), M, L, start, threads or threads_default())
        return d

    def mod_raise(self, ct_bottom: np.ndarray, L: int) -> np.ndarray:
        """mod_raise_extend_modulus (src/bootstrap.cu:37-75, :105-180): [size][1][N]
        mod q0 in NTT form -> INTT, residue v read as v - q0 when v >= q0 >> 1,
        reduced into primes 0 .. L-1, forward NTT.  [size][L][N]."""
        coef = self.ntt_inv(u64(ct_bottom))
        q0 = self.moduli[0]
        neg = coef >= np.uint64(q0 >> 1)
        mag = np.where(neg, np.uint64(q0) - coef, coef)
        out = np.empty((coef.shape[0], L, self.N), dtype=np.uint64)
        for l in range(L):
            q = np.uint64(self.moduli[l])
            r = mag[:, 0, :] % q
            out[:, l, :] = np.where(neg[:, 0, :] & (r != 0), q - r, r)
        return self.ntt_fwd(out)

    def tensor(self, a: np.ndarray, b: np.ndarray) -> np.ndarray:
        a, b = u64(a), u64(b)
        L = a.shape[-2]
        out = np.zeros((3, L, self.N), dtype=np.uint64)
        lib().orc_tensor(self._ctx, L, _p(a), _p(b), _p(out))
        return out

    def mul_poly(self, a, b, start: int = 0) -> np.ndarray:
        a, b = u64(a), u64(b)
        L = a.shape[-2]
        out = np.zeros_like(a)
        lib().orc_mul_poly(self._ctx, L, start, _p(a), _p(b), _p(out))
        return out

    def modup(self, chain_index: int, c2: np.ndarray, threads: int | None = None) -> np.ndarray:
        c2 = u64(c2)
        Ql = self.size_Ql(chain_index)
        out = np.zeros((self.beta(chain_index), Ql + self.size_P, self.N), dtype=np.uint64)
        lib().orc_modup(self._ctx, chain_index, _p(c2), _p(out), threads or threads_default())
        return out

    def ks_inner_prod(self, chain_index: int, t_mod_up: np.ndarray, key: np.ndarray) -> np.ndarray:
        t, k = u64(t_mod_up), u64(key)
        Ql = self.size_Ql(chain_index)
        out = np.zeros((2, Ql + self.size_P, self.N), dtype=np.uint64)
        lib().orc_ks_inner_prod(self._ctx, chain_index, _p(t), _p(k), k.shape[0], _p(out))
        return out

    def moddown(self, chain_index: int, cx_k: np.ndarray, threads: int | None = None) -> np.ndarray:
        cx = u64(cx_k).copy()
        Ql = self.size_Ql(chain_index)
        out = np.zeros((Ql, self.N), dtype=np.uint64)
        lib().orc_moddown(self._ctx, chain_index, _p(cx), _p(out), threads or threads_default())
        return out

    def keyswitch(self, chain_index: int, ct: np.ndarray, c2: np.ndarray, key: np.ndarray,
                  threads: int | None = None) -> np.ndarray:
        ct = u64(ct).copy()
        c2, key = u64(c2), u64(key)
        rc = lib().orc_keyswitch(self._ctx, chain_index, _p(ct), _p(c2), _p(key), key.shape[0],
                                 threads or threads_default())
        if rc != 0:
            raise ValueError("key has fewer digits than beta")
        return ct

    def multiply_and_relin(self, chain_index: int, a, b, rlk, threads: int | None = None) -> np.ndarray:
        a, b, rlk = u64(a), u64(b), u64(rlk)
        Ql = self.size_Ql(chain_index)
        out = np.zeros((2, Ql, self.N), dtype=np.uint64)
        rc = lib().orc_multiply_and_relin(self._ctx, chain_index, _p(a), _p(b), _p(rlk), rlk.shape[0],
                                          _p(out), threads or threads_default())
        if rc != 0:
            raise ValueError("key has fewer digits than beta")
        return out

    def rescale(self, chain_index: int, ct: np.ndarray, threads: int | None = None) -> np.ndarray:
        ct = u64(ct)
        size, L = ct.shape[0], ct.shape[1]
        out = np.zeros((size, L - 1, self.N), dtype=np.uint64)
        lib().orc_rescale(self._ctx, chain_index, _p(ct), size, _p(out), threads or threads_default())
        return out

    def apply_galois_ntt(self, data: np.ndarray, elt: int) -> np.ndarray:
        d = u64(data)
        L = d.size // self.N
        out = np.zeros_like(d)
        lib().orc_apply_galois_ntt(self.N, elt, _p(d), _p(out), L)
        return out

    def apply_galois(self, chain_index: int, ct: np.ndarray, elt: int, key: np.ndarray,
                     threads: int | None = None) -> np.ndarray:
        ct = u64(ct).copy()
        key = u64(key)
        rc = lib().orc_apply_galois(self._ctx, chain_index, _p(ct), elt, _p(key), key.shape[0],
                                    threads or threads_default())
        if rc != 0:
            raise ValueError("key has fewer digits than beta")
        return ct

    def hoist_rotations(self, chain_index: int, ct: np.ndarray, elts, keys,
                        threads: int | None = None) -> np.ndarray:
        ct = u64(ct)
        keys = [u64(k) for k in keys]
        Ql = self.size_Ql(chain_index)
        out = np.zeros((len(elts), 2, Ql, self.N), dtype=np.uint64)
        e = np.asarray(elts, dtype=np.uint32)
        kp = (_u64p * len(keys))(*[_p(k) for k in keys])
        rc = lib().orc_hoist_rotations(self._ctx, chain_index, _p(ct), e.ctypes.data_as(_u32p), len(elts),
                                       kp, keys[0].shape[0], _p(out), threads or threads_default())
        if rc != 0:
            raise ValueError("key has fewer digits than beta")
        return out

    def hoisting(self, chain_index: int, ct: np.ndarray, elts, keys, threads: int | None = None) -> np.ndarray:
        ct = u64(ct)
        keys = [u64(k) for k in keys]
        Ql = self.size_Ql(chain_index)
        out = np.zeros((2, Ql, self.N), dtype=np.uint64)
        e = np.asarray(elts, dtype=np.uint32)
        kp = (_u64p * len(keys))(*[_p(k) for k in keys])
        rc = lib().orc_hoisting(self._ctx, chain_index, _p(ct), e.ctypes.data_as(_u32p), len(elts), kp,
                                keys[0].shape[0], _p(out), threads or threads_default())
        if rc != 0:
            raise ValueError("key has fewer digits than beta, or no rotation")
        return out

    def kswitch_key(self, new_key, s, a, e_ntt) -> np.ndarray:
        new_key, s, a, e_ntt = u64(new_key), u64(s), u64(a), u64(e_ntt)
        dnum = self.dnum
        out = np.zeros((dnum, 2, self.size_QP, self.N), dtype=np.uint64)
        lib().orc_kswitch_key(self._ctx, _p(new_key), _p(s), _p(a), _p(e_ntt), _p(out))
        return out
