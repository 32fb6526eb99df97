"""The ciphertext operations that pyPhantom's EvalMod code is written over
(pyPhantom._GpuEngine: mod_switch_to, integer-weighted sums, multiply_and_relin
with and without the rescale, rescale_to_next, add), computed by the CPU oracle
on numpy ciphertexts.  Running the same EvalMod code over this engine gives the
residues the reference's operation sequence (src/evalmod.cu:196-335, :464-605)
produces from the oracle's primitives, which the GPU run must equal bit for bit.
Test infrastructure only."""
import numpy as np


class OCt:
    """A numpy ciphertext: data [2][|Ql|][N] uint64 in NTT form, chain index, scale."""

    def __init__(self, data, chain, scale):
        self.data, self._chain, self._scale, self._members = data, int(chain), float(scale), 1

    def chain_index(self):
        return self._chain

    def scale(self):
        return self._scale

    def set_scale(self, s):
        self._scale = float(s)

    def size(self):
        return int(self.data.shape[0])

    def _like(self, data, chain=None, scale=None):
        return OCt(data, self._chain if chain is None else chain, self._scale if scale is None else scale)


class OracleEngine:
    def __init__(self, orc, moduli, size_Q, rlk):
        self.orc, self.mods, self.Q, self.rlk = orc, [int(q) for q in moduli], int(size_Q), rlk

    def size_Ql(self, chain):
        return self.Q - (chain - 1)

    def prime(self, i):
        return self.mods[i]

    def to(self, a, chain):
        if chain == a.chain_index():
            return a
        return a._like(np.ascontiguousarray(a.data[:, :self.size_Ql(chain)]), chain=chain)

    def lincomb(self, terms, bias, chain, scale, like):
        """sum_t k_t a_t (+ bias on poly 0) in Python integers, reduced per limb."""
        L = self.size_Ql(chain)
        acc = np.zeros((like.size(), L, like.data.shape[2]), dtype=object)
        for a, k in terms:
            acc = acc + int(k) * a.data[:, :L].astype(object)
        if bias is not None:
            acc[0] = acc[0] + int(bias)
        qs = np.array(self.mods[:L], dtype=object)[None, :, None]
        return like._like((acc % qs).astype(np.uint64), chain=chain, scale=scale)

    def mul_relin(self, a, b):
        c = a.chain_index()
        assert b.chain_index() == c
        return a._like(self.orc.multiply_and_relin(c, a.data, b.data, self.rlk), scale=a.scale() * b.scale())

    def rescale(self, a):
        c = a.chain_index()
        q = self.mods[self.size_Ql(c) - 1]
        return a._like(self.orc.rescale(c, a.data), chain=c + 1, scale=a.scale() / q)

    def mul_relin_rescale(self, a, b):
        return self.rescale(self.mul_relin(a, b))

    def add(self, a, b):
        L = self.size_Ql(a.chain_index())
        qs = np.array(self.mods[:L], dtype=np.uint64)[None, :, None]
        s = a.data + b.data  # residues below 2^61: no wrap
        return a._like(np.where(s >= qs, s - qs, s))
