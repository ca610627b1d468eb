"""Pure-Python restatement of the reference TM semantics, for small cases only.

Written independently of oracle/ytm_oracle.c (own Philox, own site mapping, own loops)
so that the C oracle is checked against a second reading of the reference:
  encode_batch          src/cutm/cuda/kernel.cu:76-152
  pack_clauses          src/cutm/cuda/kernel.cu:155-204
  clause_match          src/cutm/cuda/kernel.cu:207-216
  fast_eval             src/cutm/cuda/kernel.cu:255-282
  select_active         src/cutm/cuda/kernel.cu:285-316
  calc_class_sums_infer src/cutm/cuda/kernel.cu:319-343
  transform(_patchwise) src/cutm/cuda/kernel.cu:346-394
  clause_update & fb    src/cutm/cuda/kernel.cu:397-613
  per-sample driver     src/cutm/base.py:305-357
"""
from __future__ import annotations

import numpy as np

MASK32 = 0xFFFFFFFF


def philox(ctr, key, rounds=10):
    """Philox4x32 (Salmon et al., SC'11): multipliers 0xD2511F53 / 0xCD9E8D57, Weyl key
    increments 0x9E3779B9 / 0xBB67AE85."""
    c0, c1, c2, c3 = (int(v) & MASK32 for v in ctr)
    k0, k1 = (int(v) & MASK32 for v in key)
    for r in range(rounds):
        if r:
            k0 = (k0 + 0x9E3779B9) & MASK32
            k1 = (k1 + 0xBB67AE85) & MASK32
        p0 = 0xD2511F53 * c0
        p1 = 0xCD9E8D57 * c2
        c0, c1, c2, c3 = ((p1 >> 32) ^ c1 ^ k0) & MASK32, p1 & MASK32, ((p0 >> 32) ^ c3 ^ k1) & MASK32, p0 & MASK32
    return (c0, c1, c2, c3)


def u_of_word(z: int) -> float:
    return float(np.float32((z >> 8) + 1) * np.float32(2.0 ** -24))


class Stream:
    """The canonical draw sites (counter mode) or an injected per-sample block."""

    SEL, CK, LIT, INIT = 1, 2, 3, 4

    def __init__(self, seed, C, K, P, L, W, inject=None):
        self.key = (seed & MASK32, (seed >> 32) & MASK32)
        self.C, self.K, self.P, self.L, self.W = C, K, P, L, W
        self.inject = inject
        self.block = C * P + 2 * C * K + C * K * L

    def _words(self, t, c, tag, site):
        return philox((t & MASK32, c, (tag << 28) | ((t >> 32) & 0x0FFFFFFF), site), self.key)

    def sel(self, i, t, c, r):
        if self.inject is not None:
            return float(self.inject[i * self.block + c * self.P + (r - 1)])
        return u_of_word(self._words(t, c, self.SEL, (r - 1) // 4)[(r - 1) % 4])

    def q(self, i, t, c, k):
        if self.inject is not None:
            return float(self.inject[i * self.block + self.C * self.P + c * self.K + k])
        return u_of_word(self._words(t, c, self.CK, k)[0])

    def upd(self, i, t, c, k):
        if self.inject is not None:
            return float(self.inject[i * self.block + self.C * self.P + self.C * self.K + c * self.K + k])
        return u_of_word(self._words(t, c, self.CK, k)[1])

    def lit(self, i, t, c, k, l):
        if self.inject is not None:
            return float(self.inject[i * self.block + self.C * self.P + 2 * self.C * self.K + (c * self.K + k) * self.L + l])
        w, b = divmod(l, 32)
        q = 0
        for g in range(6):
            z = self._words(t, c, self.LIT, (k * self.W + w) * 6 + g)
            for i4 in range(4):
                q |= ((z[i4] >> b) & 1) << (23 - 4 * g - i4)
        return float(np.float32(q + 1) * np.float32(2.0 ** -24))


class PyTM:
    def __init__(self, C, K, T, s_inv, q_prob, dim, patch_dim, *, n_states=256, maxinc=None, append_negated=True,
                 encode_loc=True, coalesced=True, negative_polarity=True, init_neg_weights=True, seed=0):
        self.C, self.K, self.T = C, K, T
        self.s_inv, self.q_prob = s_inv, q_prob
        self.dim, self.patch_dim = dim, patch_dim
        self.append_negated, self.encode_loc = append_negated, encode_loc
        self.coalesced, self.negative_polarity = coalesced, negative_polarity
        self.n_states = n_states
        base = patch_dim[0] * patch_dim[1] * dim[2]
        if encode_loc:
            base += (dim[0] - patch_dim[0]) + (dim[1] - patch_dim[1])
        self.L = 2 * base if append_negated else base
        self.W = (self.L - 1) // 32 + 1
        self.P = (dim[0] - patch_dim[0] + 1) * (dim[1] - patch_dim[1] + 1)
        self.maxinc = self.L if maxinc is None else maxinc
        self.seed = seed
        self.step = 0
        self.ta = [[n_states // 2] * self.L for _ in range(C)]
        per_bank = C // (1 if coalesced else K)
        self.per_bank = per_bank
        st = Stream(seed, C, K, self.P, self.L, self.W)
        self.w = [[0.0] * K for _ in range(C)]
        for c in range(C):
            for k in range(K):
                if coalesced:
                    v = 1.0
                    if init_neg_weights:
                        v = 1.0 - 2.0 * float(st._words(0, c, Stream.INIT, k)[0] & 1)
                elif k == c // per_bank:
                    v = -1.0 if (init_neg_weights and c % per_bank >= per_bank // 2) else 1.0
                else:
                    v = 0.0
                self.w[c][k] = v
        self.pw = [[0] * self.P for _ in range(C)]

    # -------------------------------------------------------------- encode
    def encode(self, X):
        d0, d1, d2 = self.dim
        p0, p1 = self.patch_dim
        N = len(X)
        out = np.zeros((N, self.P, self.W), dtype=np.uint32)
        half = self.L // 2
        for e in range(N):
            for patch in range(self.P):
                bits = [0] * (self.W * 32)
                py, px = patch // (d0 - p0 + 1), patch % (d0 - p0 + 1)
                if self.append_negated:
                    for l in range(half, self.L):
                        bits[l] = 1
                for l in range(py):
                    bits[l] = 1
                    if self.append_negated:
                        bits[l + half] = 0
                for l in range(px):
                    bits[(d1 - p1) + l] = 1
                    if self.append_negated:
                        bits[(d1 - p1) + l + half] = 0
                for y in range(py, py + p1):
                    for x in range(px, px + p0):
                        for z in range(d2):
                            if X[e][y * d0 * d2 + x * d2 + z] > 0:
                                pos = (y - py) * p0 * d2 + (x - px) * d2 + z
                                if self.encode_loc:
                                    pos += (d1 - p1) + (d0 - p0)
                                bits[pos] = 1
                                if self.append_negated:
                                    bits[pos + half] = 0
                for w in range(self.W):
                    out[e, patch, w] = sum(bits[w * 32 + b] << b for b in range(32))
        return out

    # -------------------------------------------------------------- evaluation
    def _includes(self, c):
        return [l for l in range(self.L) if self.ta[c][l] > self.n_states // 2]

    @staticmethod
    def _bit(x, l):
        return (int(x[l // 32]) >> (l % 32)) & 1

    def _match(self, inc, x):
        return all(self._bit(x, l) for l in inc)

    def score(self, encX):
        out = np.zeros((len(encX), self.K), dtype=np.float32)
        incs = [self._includes(c) for c in range(self.C)]
        for e in range(len(encX)):
            s = [0] * self.K
            for c in range(self.C):
                if not incs[c]:
                    continue
                if any(self._match(incs[c], encX[e][p]) for p in range(self.P)):
                    for k in range(self.K):
                        s[k] += int(self.w[c][k])
            out[e] = s
        return out

    def transform(self, encX, patchwise=False):
        incs = [self._includes(c) for c in range(self.C)]
        N = len(encX)
        if patchwise:
            out = np.zeros((N, self.C, self.P), dtype=np.uint32)
            for e in range(N):
                for c in range(self.C):
                    for p in range(self.P):
                        out[e, c, p] = 1 if not incs[c] else int(self._match(incs[c], encX[e][p]))
            return out
        out = np.zeros((N, self.C), dtype=np.uint32)
        for e in range(N):
            for c in range(self.C):
                out[e, c] = 1 if not incs[c] else int(any(self._match(incs[c], encX[e][p]) for p in range(self.P)))
        return out

    # -------------------------------------------------------------- training
    def fit(self, encX, encY, drop=None, inject=None):
        C, K, P, L = self.C, self.K, self.P, self.L
        drop = [0] * C if drop is None else [int(v) for v in drop]
        st = Stream(self.seed, C, K, P, L, self.W, inject)
        T = np.float32(self.T)
        updated = 0
        for i in range(len(encX)):
            t = self.step + i
            x = encX[i]
            incs = [self._includes(c) for c in range(C)]
            ninc = [len(v) for v in incs]
            cs = [0] * K
            sel = [-1] * C
            for c in range(C):
                if drop[c] == 1:
                    continue
                count = 0
                for p in range(P):
                    out = 1 if ninc[c] == 0 else int(self._match(incs[c], x[p]))
                    if out:
                        count += 1
                        if np.float32(st.sel(i, t, c, count)) < np.float32(1.0) / np.float32(count):
                            sel[c] = p
                if sel[c] != -1:
                    self.pw[c][sel[c]] += 1
                    ks = range(K) if self.coalesced else [c // self.per_bank]
                    for k in ks:
                        cs[k] += int(self.w[c][k])
            v, tgt, prob = [], [], []
            for k in range(K):
                csf = np.float32(cs[k])
                vk = T if csf > T else (-T if csf < -T else csf)
                y = int(encY[i][k])
                v.append(vk)
                tgt.append(1 - 2 * int(vk > np.float32(y)))
                prob.append((float(y) - float(vk)) / (2.0 * float(y)))
            for c in range(C):
                if drop[c] == 1:
                    continue
                o = sel[c] > -1
                patch = x[sel[c]] if o else None
                ks = range(K) if self.coalesced else [c // self.per_bank]
                touched = False
                for k in ks:
                    if tgt[k] == -1 and st.q(i, t, c, k) > self.q_prob:
                        continue
                    wv = self.w[c][k]
                    sign = (wv >= 0) - (wv < 0)
                    upd = st.upd(i, t, c, k) <= prob[k]
                    small = o and ninc[c] <= self.maxinc
                    t1a = tgt[k] * sign > 0 and small
                    t1b = tgt[k] * sign > 0 and not small
                    t2 = tgt[k] * sign < 0 and o
                    if not upd:
                        continue
                    row = self.ta[c]
                    if t1a:
                        self.w[c][k] = float(np.float32(wv) + np.float32(sign))
                        for l in range(L):
                            b = self._bit(patch, l)
                            if b == 1 and row[l] < self.n_states:
                                row[l] += 1
                            elif b == 0 and row[l] > 0 and st.lit(i, t, c, k, l) <= self.s_inv:
                                row[l] -= 1
                        touched = True
                    elif t1b:
                        for l in range(L):
                            if row[l] > 0 and st.lit(i, t, c, k, l) <= self.s_inv:
                                row[l] -= 1
                        touched = True
                    elif t2:
                        nw = float(np.float32(wv) - np.float32(sign))
                        if not self.negative_polarity and nw < 1:
                            nw = 1.0
                        self.w[c][k] = nw
                        for l in range(L):
                            if self._bit(patch, l) == 0:
                                row[l] += 1
                        touched = True
                updated += int(touched)
        self.step += len(encX)
        return updated

    # -------------------------------------------------------------- views
    def ta_array(self):
        return np.array(self.ta, dtype=np.uint32)

    def w_array(self):
        return np.array(self.w, dtype=np.float32)

    def pw_array(self):
        return np.array(self.pw, dtype=np.int32)
