"""ctypes binding of libphantom_amd.so (the C ABI declared in include/phantom_amd.h).

This is the only way Python reaches the HIP kernels.  It fails loudly when the
library is missing: there is no CPU fallback anywhere in the product.

Device buffers are torch tensors of dtype torch.uint64 on a ROCm device; only
their data pointers cross the boundary.  Streams default to torch's current
stream on the tensor's device.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libphantom_amd.so")

PFA_OK = 0
PFA_ERR_INVALID_ARGUMENT = 1
PFA_ERR_LOGIC = 2
PFA_ERR_RUNTIME = 3

_vp, _sz, _u64, _u32, _i32 = C.c_void_p, C.c_size_t, C.c_uint64, C.c_uint32, C.c_int
_u64p = C.POINTER(C.c_uint64)

# name -> (restype, argtypes); mirrors include/phantom_amd.h one to one
SIGNATURES = {
    "pfa_last_error": (C.c_char_p, []),
    "pfa_abi_version": (_i32, []),
    "pfa_create_coeff_modulus": (_i32, [_u64, C.POINTER(C.c_int), _sz, _u64p]),
    "pfa_context_create": (_i32, [_u64, _u64p, _sz, _sz, _i32, C.POINTER(_vp)]),
    "pfa_context_destroy": (None, [_vp]),
    "pfa_context_roots": (_i32, [_vp, _u64p]),
    "pfa_synchronize": (_i32, [_vp, _vp]),
    "pfa_ntt_single_launch": (_i32, [_vp, _sz, _sz, C.POINTER(C.c_int)]),
    "pfa_stream_copy": (_i32, [_vp, _vp, _sz, _sz, _vp]),
    "pfa_ntt_forward": (_i32, [_vp, _vp, _sz, _sz, _sz, _vp]),
    "pfa_ntt_inverse": (_i32, [_vp, _vp, _sz, _sz, _sz, _vp]),
    "pfa_modup": (_i32, [_vp, _sz, _vp, _vp, _vp]),
    "pfa_ks_inner_prod": (_i32, [_vp, _sz, _vp, _vp, _sz, _vp, _vp]),
    "pfa_moddown": (_i32, [_vp, _sz, _vp, _vp, _vp]),
    "pfa_keyswitch": (_i32, [_vp, _sz, _vp, _vp, _vp, _sz, _vp]),
    "pfa_tensor": (_i32, [_vp, _sz, _vp, _vp, _vp, _vp]),
    "pfa_multiply_and_relin": (_i32, [_vp, _sz, _vp, _vp, _vp, _sz, _vp, _vp]),
    "pfa_relinearize": (_i32, [_vp, _sz, _vp, _vp, _sz, _vp, _vp]),
    "pfa_rescale": (_i32, [_vp, _sz, _vp, _sz, _vp, _vp]),
    "pfa_rescale_noalloc": (_i32, [_vp, _sz, _vp, _sz, _vp, _vp]),
    "pfa_multiply_relin_rescale": (_i32, [_vp, _sz, _vp, _vp, _vp, _sz, _vp, _vp]),
    "pfa_relinearize_rescale": (_i32, [_vp, _sz, _vp, _vp, _sz, _vp, _vp]),
    "pfa_multiply_and_relin_batch": (_i32, [_vp, _sz, _sz, _vp, _vp, _vp, _sz, _vp, _vp]),
    "pfa_multiply_relin_rescale_batch": (_i32, [_vp, _sz, _sz, _vp, _vp, _vp, _sz, _vp, _vp]),
    "pfa_galois_elt_from_step": (_i32, [_i32, _u64, C.POINTER(C.c_uint32)]),
    "pfa_apply_galois_ntt": (_i32, [_vp, _u32, _vp, _vp, _sz, _vp]),
    "pfa_apply_galois": (_i32, [_vp, _sz, _vp, _u32, _vp, _sz, _vp]),
    "pfa_hoist_rotations": (_i32, [_vp, _sz, _vp, C.POINTER(C.c_uint32), _sz, C.POINTER(_vp), _sz, _vp, _vp]),
    "pfa_hoisting": (_i32, [_vp, _sz, _vp, C.POINTER(C.c_uint32), _sz, C.POINTER(_vp), _sz, _vp, _vp]),
    "pfa_kswitch_key": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "pfa_poly_add": (_i32, [_vp, _vp, _vp, _vp, _sz, _sz, _vp]),
    "pfa_poly_sub": (_i32, [_vp, _vp, _vp, _vp, _sz, _sz, _vp]),
    "pfa_poly_mul": (_i32, [_vp, _vp, _vp, _vp, _sz, _sz, _vp]),
    "pfa_poly_negate": (_i32, [_vp, _vp, _vp, _sz, _sz, _vp]),
    "pfa_ct_multiply_plain": (_i32, [_vp, _vp, _sz, _vp, _vp, _sz, _vp]),
    "pfa_poly_from_signed": (_i32, [_vp, _vp, _vp, _sz, _sz, _vp]),
    "pfa_ckks_encode": (_i32, [_vp, _vp, _sz, C.c_double, _vp, _sz, _vp]),
    "pfa_ckks_decode": (_i32, [_vp, _vp, _sz, C.c_double, _vp, _vp]),
    "pfa_ckks_encode_coeffs": (_i32, [_vp, _vp, _sz, C.c_double, _vp, _vp]),
    "pfa_expand_signed": (_i32, [_vp, _vp, _sz, _vp, _sz, _sz, _vp]),
    "pfa_bsgs_mac": (_i32, [_vp, _sz, C.POINTER(_vp), C.POINTER(_vp), _sz, _sz, C.POINTER(_vp), _vp]),
    "pfa_bsgs_tile_plaintexts": (_i32, [_vp, _sz, _vp, _sz, _vp, _sz, _sz, _vp]),
    "pfa_bsgs_mac_tiled": (_i32, [_vp, _sz, _vp, C.POINTER(_vp), _sz, _sz, C.POINTER(_vp), _vp]),
    "pfa_bsgs_tiled_size": (_i32, [_vp, _sz, _sz, C.POINTER(_sz)]),
    "pfa_bsgs_babies": (_i32, [_vp, _sz, _vp, _sz, C.POINTER(_vp), _sz, _vp, _vp]),
    "pfa_rotate_batch": (_i32, [_vp, _sz, _sz, _vp, C.POINTER(C.c_uint32), C.POINTER(_vp), _sz, _vp, _vp]),
    "pfa_bsgs_giants": (_i32, [_vp, _sz, _vp, _sz, _i32, _vp, _sz, _vp, _vp]),
    "pfa_bsgs_apply_giants": (_i32, [_vp, _sz, _vp, C.POINTER(_vp), _sz, _sz, _vp, _sz, _vp, _vp]),
    "pfa_mod_raise": (_i32, [_vp, _vp, _sz, _vp, _vp]),
    "pfa_ct_lincomb": (_i32, [_vp, _sz, _sz, _sz, _vp, _vp, _vp, _sz, _vp, _vp, _vp]),
}


class PhantomError(RuntimeError):
    pass


_lib = None


def lib():
    """Load libphantom_amd.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"libphantom_amd.so not found at {LIB_PATH}: build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'` (there is no CPU fallback)")
        # torch first: its wheel carries its own HIP runtime, which torch loads as
        # "libamdhip64.so".  Loaded after it, this library binds to that same
        # runtime (soname libamdhip64.so.7); loaded before, it brings in the
        # system copy and torch then starts a second runtime that sees no device.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> None:
    """Raise the Python counterpart of the reference's exception class."""
    if rc == PFA_OK:
        return
    msg = lib().pfa_last_error().decode(errors="replace")
    if rc == PFA_ERR_INVALID_ARGUMENT:
        raise ValueError(msg)  # std::invalid_argument under pybind11
    raise PhantomError(msg)    # std::logic_error / std::runtime_error -> RuntimeError


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))


def ptr(t) -> int:
    """Device pointer of a contiguous torch uint64 tensor (None -> NULL)."""
    if t is None:
        return None
    import torch

    if t.device.type != "cuda":
        raise ValueError("expected a device tensor")
    if t.dtype != torch.uint64:
        raise ValueError(f"expected torch.uint64, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError("expected a contiguous tensor")
    return t.data_ptr()


# torch's default stream reports handle 0 and is HIP's legacy default stream;
# the C ABI reads a NULL stream as hipStreamPerThread (the reference's
# cudaStreamPerThread), a different stream that the legacy one synchronizes
# with implicitly.  A torch kernel followed by the library's work on those two
# streams then cost ~70 us of GPU time per switch (and a bootstrap with one
# such switch ~2 ms), so the default stream is passed as hipStreamLegacy.
HIP_STREAM_LEGACY = 1


def stream_handle(stream) -> int:
    """The hipStream_t to pass for a torch stream (its handle, or
    hipStreamLegacy for torch's default stream)."""
    return stream.cuda_stream or HIP_STREAM_LEGACY


def stream_of(t=None):
    import torch

    dev = t.device if t is not None else torch.device("cuda", torch.cuda.current_device())
    return stream_handle(torch.cuda.current_stream(dev))


def stream_copy(dst, src, workgroups: int = 0, stream=None):
    """Streaming copy of a uint64 tensor into another of the same size (the
    achievable-bandwidth reference of the NTT's measurement)."""
    if dst.numel() != src.numel():
        raise ValueError("copy between tensors of different sizes")
    call("pfa_stream_copy", ptr(dst), ptr(src), src.numel(), workgroups, stream or stream_of(src))


def create_coeff_modulus(poly_degree: int, bit_sizes) -> list[int]:
    bits = (C.c_int * len(bit_sizes))(*bit_sizes)
    out = (C.c_uint64 * len(bit_sizes))()
    call("pfa_create_coeff_modulus", poly_degree, bits, len(bit_sizes), out)
    return [int(x) for x in out]


def galois_elt_from_step(step: int, poly_degree: int) -> int:
    e = C.c_uint32(0)
    call("pfa_galois_elt_from_step", step, poly_degree, C.byref(e))
    return int(e.value)


class NativeContext:
    """Owns a pfa_context: the chain, NTT tables and RNS constants on one device."""

    def __init__(self, poly_degree: int, moduli, special_size: int, device: int = 0):
        self.N = int(poly_degree)
        self.moduli = [int(m) for m in moduli]
        self.size_QP = len(self.moduli)
        self.size_P = int(special_size)
        self.size_Q = self.size_QP - self.size_P
        self.device = device
        arr = (C.c_uint64 * self.size_QP)(*self.moduli)
        h = C.c_void_p()
        call("pfa_context_create", self.N, arr, self.size_QP, self.size_P, device, C.byref(h))
        self._h = h

    @property
    def handle(self):
        return self._h

    def close(self):
        if getattr(self, "_h", None):
            lib().pfa_context_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def roots(self) -> list[int]:
        out = (C.c_uint64 * self.size_QP)()
        call("pfa_context_roots", self._h, out)
        return [int(x) for x in out]

    def size_Ql(self, chain_index: int) -> int:
        return self.size_Q - (chain_index - 1)

    def beta(self, chain_index: int) -> int:
        return -(-self.size_Ql(chain_index) // self.size_P)

    @property
    def dnum(self) -> int:
        return self.size_Q // self.size_P

    # ---- raw entry points (device tensors in, device tensors out) ----
    def ntt_forward(self, data, M: int, L: int, start: int = 0, stream=None):
        call("pfa_ntt_forward", self._h, ptr(data), M, L, start, stream or stream_of(data))

    def ntt_inverse(self, data, M: int, L: int, start: int = 0, stream=None):
        call("pfa_ntt_inverse", self._h, ptr(data), M, L, start, stream or stream_of(data))

    def ntt_single_launch(self, M: int, L: int) -> bool:
        """True if an NTT of M x L limbs runs as one launch (intermediate in L2)."""
        out = C.c_int(0)
        call("pfa_ntt_single_launch", self._h, M, L, C.byref(out))
        return bool(out.value)

    def synchronize(self, stream=None):
        """Waits for `stream` (default: torch's current stream on the context's
        device) and raises RuntimeError if a kernel of this context recorded an
        error on the device (a single-launch NTT that did not finish, or a
        key-switch inner product whose split item ran on two XCDs)."""
        if stream is None:
            import torch

            stream = stream_handle(torch.cuda.current_stream(self.device))
        call("pfa_synchronize", self._h, stream)

    def modup(self, chain_index, c2, out, stream=None):
        call("pfa_modup", self._h, chain_index, ptr(c2), ptr(out), stream or stream_of(c2))

    def ks_inner_prod(self, chain_index, t_mod_up, key, cx, stream=None):
        call("pfa_ks_inner_prod", self._h, chain_index, ptr(t_mod_up), ptr(key), key.shape[0], ptr(cx),
             stream or stream_of(key))

    def moddown(self, chain_index, cx_k, out, stream=None):
        call("pfa_moddown", self._h, chain_index, ptr(cx_k), ptr(out), stream or stream_of(cx_k))

    def keyswitch(self, chain_index, ct, c2, key, stream=None):
        call("pfa_keyswitch", self._h, chain_index, ptr(ct), ptr(c2), ptr(key), key.shape[0],
             stream or stream_of(ct))

    def tensor(self, chain_index, a, b, out, stream=None):
        call("pfa_tensor", self._h, chain_index, ptr(a), ptr(b), ptr(out), stream or stream_of(a))

    def multiply_and_relin(self, chain_index, a, b, rlk, out, stream=None):
        call("pfa_multiply_and_relin", self._h, chain_index, ptr(a), ptr(b), ptr(rlk), rlk.shape[0], ptr(out),
             stream or stream_of(a))

    def relinearize(self, chain_index, ct3, rlk, out, stream=None):
        call("pfa_relinearize", self._h, chain_index, ptr(ct3), ptr(rlk), rlk.shape[0], ptr(out),
             stream or stream_of(ct3))

    def multiply_relin_rescale(self, chain_index, a, b, rlk, out, stream=None):
        call("pfa_multiply_relin_rescale", self._h, chain_index, ptr(a), ptr(b), ptr(rlk), rlk.shape[0], ptr(out),
             stream or stream_of(a))

    def multiply_and_relin_batch(self, chain_index, count, a, b, rlk, out, stream=None):
        call("pfa_multiply_and_relin_batch", self._h, chain_index, count, ptr(a), ptr(b), ptr(rlk), rlk.shape[0],
             ptr(out), stream or stream_of(a))

    def multiply_relin_rescale_batch(self, chain_index, count, a, b, rlk, out, stream=None):
        call("pfa_multiply_relin_rescale_batch", self._h, chain_index, count, ptr(a), ptr(b), ptr(rlk), rlk.shape[0],
             ptr(out), stream or stream_of(a))

    def relinearize_rescale(self, chain_index, ct3, rlk, out, stream=None):
        call("pfa_relinearize_rescale", self._h, chain_index, ptr(ct3), ptr(rlk), rlk.shape[0], ptr(out),
             stream or stream_of(ct3))

    def rescale(self, chain_index, ct, out, stream=None):
        call("pfa_rescale", self._h, chain_index, ptr(ct), ct.shape[0], ptr(out), stream or stream_of(ct))

    def rescale_noalloc(self, chain_index, ct, out, stream=None):
        """pfa_rescale_noalloc: the same residues as rescale, with no device
        allocation (a static per-device scratch; see include/phantom_amd.h)."""
        call("pfa_rescale_noalloc", self._h, chain_index, ptr(ct), ct.shape[0], ptr(out), stream or stream_of(ct))

    def apply_galois_ntt(self, elt, src, dst, L, stream=None):
        call("pfa_apply_galois_ntt", self._h, elt, ptr(src), ptr(dst), L, stream or stream_of(src))

    def apply_galois(self, chain_index, ct, elt, key, stream=None):
        call("pfa_apply_galois", self._h, chain_index, ptr(ct), elt, ptr(key), key.shape[0],
             stream or stream_of(ct))

    def hoist_rotations(self, chain_index, ct, elts, keys, out, stream=None):
        n = len(elts)
        e = (C.c_uint32 * n)(*elts)
        kp = (C.c_void_p * n)(*[ptr(k) for k in keys])
        call("pfa_hoist_rotations", self._h, chain_index, ptr(ct), e, n, kp, keys[0].shape[0], ptr(out),
             stream or stream_of(ct))

    def hoisting(self, chain_index, ct, elts, keys, out, stream=None):
        n = len(elts)
        e = (C.c_uint32 * n)(*elts)
        kp = (C.c_void_p * n)(*[ptr(k) for k in keys])
        call("pfa_hoisting", self._h, chain_index, ptr(ct), e, n, kp, keys[0].shape[0], ptr(out),
             stream or stream_of(ct))

    def kswitch_key(self, new_key, s, a, e, out, stream=None):
        call("pfa_kswitch_key", self._h, ptr(new_key), ptr(s), ptr(a), ptr(e), ptr(out), stream or stream_of(s))

    def poly_add(self, a, b, out, L, start=0, stream=None):
        call("pfa_poly_add", self._h, ptr(a), ptr(b), ptr(out), L, start, stream or stream_of(a))

    def poly_sub(self, a, b, out, L, start=0, stream=None):
        call("pfa_poly_sub", self._h, ptr(a), ptr(b), ptr(out), L, start, stream or stream_of(a))

    def poly_mul(self, a, b, out, L, start=0, stream=None):
        call("pfa_poly_mul", self._h, ptr(a), ptr(b), ptr(out), L, start, stream or stream_of(a))

    def ct_multiply_plain(self, ct, pt, out, L, stream=None):
        """out[k] = ct[k] * pt over limbs 0..L-1 for every poly of ct [size][L][N]."""
        if ct.shape[0] != out.shape[0] or not ct.is_contiguous() or not out.is_contiguous():
            raise ValueError("ct and out must be contiguous [size][L][N] tensors of one size")
        call("pfa_ct_multiply_plain", self._h, ptr(ct), ct.shape[0], ptr(pt), ptr(out), L, stream or stream_of(ct))

    def poly_negate(self, a, out, L, start=0, stream=None):
        call("pfa_poly_negate", self._h, ptr(a), ptr(out), L, start, stream or stream_of(a))

    def ckks_encode(self, values_c128, scale, out, L, stream=None):
        """values_c128: complex128 device tensor [<= N/2]; out: uint64 [L][N]."""
        import torch

        if values_c128.dtype != torch.complex128 or values_c128.device.type != "cuda":
            raise ValueError("expected a complex128 device tensor")
        v = values_c128.contiguous()
        call("pfa_ckks_encode", self._h, v.data_ptr(), v.numel(), float(scale), ptr(out), L,
             stream or stream_of(out))

    def ckks_decode(self, plain, L, scale, out_c128, stream=None):
        import torch

        if out_c128.dtype != torch.complex128 or not out_c128.is_contiguous():
            raise ValueError("expected a contiguous complex128 device tensor")
        call("pfa_ckks_decode", self._h, ptr(plain), L, float(scale), out_c128.data_ptr(),
             stream or stream_of(plain))

    def ckks_encode_coeffs(self, values_c128, scale, out_i64, stream=None):
        """values_c128: complex128 device tensor [<= N/2]; out_i64: int64 [N] (signed coefficients)."""
        import torch

        if values_c128.dtype != torch.complex128 or values_c128.device.type != "cuda":
            raise ValueError("expected a complex128 device tensor")
        if out_i64.dtype != torch.int64 or not out_i64.is_contiguous():
            raise ValueError("expected a contiguous int64 device tensor")
        v = values_c128.contiguous()
        call("pfa_ckks_encode_coeffs", self._h, v.data_ptr(), v.numel(), float(scale), out_i64.data_ptr(),
             stream or stream_of(out_i64))

    def expand_signed(self, coeffs_i64, n, out, L, start=0, stream=None):
        """coeffs_i64: int64 [n][N]; out: uint64 [n][L][N] residues (coefficient form)."""
        import torch

        if coeffs_i64.dtype != torch.int64 or not coeffs_i64.is_contiguous():
            raise ValueError("expected a contiguous int64 device tensor")
        call("pfa_expand_signed", self._h, coeffs_i64.data_ptr(), n, ptr(out), L, start,
             stream or stream_of(out))

    def bsgs_mac(self, chain_index, pts, babies, outs, stream=None):
        """outs[g] = sum_b pts[g * M + b] * babies[b] (M = len(babies), G = len(outs)).
        Entries are device tensors or raw device addresses (ints); with addresses
        only, pass `stream`."""
        M, G = len(babies), len(outs)
        if len(pts) != M * G:
            raise ValueError("need len(babies) * len(outs) plaintexts")
        addr = lambda t: t if isinstance(t, int) else ptr(t)
        pp = (C.c_void_p * (M * G))(*[addr(t) for t in pts])
        bp = (C.c_void_p * M)(*[addr(t) for t in babies])
        op = (C.c_void_p * G)(*[addr(t) for t in outs])
        if stream is None:
            first = next((t for t in list(outs) + list(babies) if not isinstance(t, int)), None)
            stream = stream_of(first) if first is not None else None
        call("pfa_bsgs_mac", self._h, chain_index, pp, bp, M, G, op, stream)

    def bsgs_tile_plaintexts(self, chain_index, src, n, tiled, d0, D, stream=None):
        """src [n][Ql][N] -> positions d0 .. d0+n-1 of the tiled set `tiled` of D plaintexts."""
        call("pfa_bsgs_tile_plaintexts", self._h, chain_index, ptr(src), n, ptr(tiled), d0, D,
             stream or stream_of(src))

    def bsgs_tiled_size(self, chain_index, D) -> int:
        """Bytes of a tiled set of D plaintexts at chain_index."""
        n = C.c_size_t(0)
        call("pfa_bsgs_tiled_size", self._h, chain_index, D, C.byref(n))
        return int(n.value)

    def bsgs_mac_tiled(self, chain_index, tiled, babies, outs, stream=None):
        """bsgs_mac with the len(babies) * len(outs) plaintexts in one tiled set."""
        M, G = len(babies), len(outs)
        addr = lambda t: t if isinstance(t, int) else ptr(t)
        bp = (C.c_void_p * M)(*[addr(t) for t in babies])
        op = (C.c_void_p * G)(*[addr(t) for t in outs])
        call("pfa_bsgs_mac_tiled", self._h, chain_index, ptr(tiled), bp, M, G, op, stream or stream_of(tiled))

    def rotate_batch(self, chain_index, inp, elts, keys, out, stream=None):
        """out[i] = rotate(inp[i], elts[i]) with keys[i]; inp, out [count][2][L][N]."""
        n = len(elts)
        if len(keys) != n or n == 0:
            raise ValueError("one key per Galois element, at least one")
        ep = (C.c_uint32 * n)(*[int(e) for e in elts])
        kp = (C.c_void_p * n)(*[ptr(k) for k in keys])
        call("pfa_rotate_batch", self._h, chain_index, n, ptr(inp), ep, kp, keys[0].shape[0], ptr(out),
             stream or stream_of(inp))

    def bsgs_babies(self, chain_index, ct, M, keys, out, stream=None):
        """out[b] = babies[b] for 0 <= b < M (out[0] = ct, then chained
        power-of-two rotations); keys[k] is the Galois key of step 2^k for every 2^k < M."""
        kp = (C.c_void_p * max(len(keys), 1))(*[ptr(k) for k in keys])
        dnum = keys[0].shape[0] if keys else 0
        call("pfa_bsgs_babies", self._h, chain_index, ptr(ct), M, kp, dnum, ptr(out), stream or stream_of(ct))

    def bsgs_giants(self, chain_index, partials, G, step, key, out, stream=None):
        """Horner over the giant partials (overwritten) with rotation `step`, then rescale into out."""
        call("pfa_bsgs_giants", self._h, chain_index, ptr(partials), G, step, ptr(key) if key is not None else None,
             key.shape[0] if key is not None else 0, ptr(out), stream or stream_of(partials))

    def bsgs_apply_giants(self, chain_index, tiled, babies, G, key, out, stream=None):
        """Accumulation of the G giants' partials (tiled plaintext set), Horner
        rotations by M = len(babies) and the rescale into out [2][Ql-1][N]."""
        M = len(babies)
        addr = lambda t: t if isinstance(t, int) else ptr(t)
        bp = (C.c_void_p * M)(*[addr(t) for t in babies])
        call("pfa_bsgs_apply_giants", self._h, chain_index, ptr(tiled), bp, M, G,
             ptr(key) if key is not None else None, key.shape[0] if key is not None else 0, ptr(out),
             stream or stream_of(tiled))

    def ct_lincomb(self, L, ins, consts, out, bias=None, stream=None, ct_size=None):
        """out [size][L][N] = sum_t consts[t] ins[t] (+ bias on poly 0 of each
        ciphertext of ct_size polys, default size); ins are [size][L_t][N]
        tensors with L_t >= L; consts Python ints in int64 range, bias a Python
        int in the signed 128-bit range or None."""
        n = len(ins)
        size = out.shape[0]
        for t in ins:
            if t.shape[0] != size or t.shape[2] != out.shape[2] or not t.is_contiguous():
                raise ValueError("inputs must be contiguous [size][L_t][N] like the output")
        ip = (C.c_void_p * max(n, 1))(*[ptr(t) for t in ins])
        il = (C.c_size_t * max(n, 1))(*[t.shape[1] for t in ins])
        kc = (C.c_int64 * max(n, 1))(*[int(k) for k in consts])
        bp = None
        if bias is not None:
            b = int(bias)
            if not -(1 << 127) <= b < (1 << 127):
                raise ValueError("bias out of the signed 128-bit range")
            b &= (1 << 128) - 1
            bp = (C.c_uint64 * 2)(b & 0xFFFFFFFFFFFFFFFF, b >> 64)
        call("pfa_ct_lincomb", self._h, L, size, ct_size or size, ip, il, kc, n, bp, ptr(out),
             stream or stream_of(out))

    def mod_raise(self, ct_bottom, out, stream=None):
        """ct_bottom [size][1][N] mod q0 -> out [size][|Q|][N], centred lift (NTT form)."""
        call("pfa_mod_raise", self._h, ptr(ct_bottom), ct_bottom.shape[0], ptr(out), stream or stream_of(out))

    def poly_from_signed(self, coeffs_i64, out, L, start=0, stream=None):
        import torch

        if coeffs_i64.dtype != torch.int64 or coeffs_i64.device.type != "cuda":
            raise ValueError("expected an int64 device tensor")
        call("pfa_poly_from_signed", self._h, coeffs_i64.data_ptr(), ptr(out), L, start,
             stream or stream_of(out))
