"""Hand-derived known answers for the oracle: each expected value below is worked out
from the reference source by hand (cited), not by re-running a restatement."""
import numpy as np
import pytest


def bits_to_words(bits, W):
    out = np.zeros(W, dtype=np.uint32)
    for b in bits:
        out[b // 32] |= np.uint32(1) << np.uint32(b % 32)
    return out


# ------------------------------------------------------------------ encode (kernel.cu:76-152)
def test_encode_single_pixel_conv(oracle_mod):
    # dim (4,4,1), patch (2,2): L = (2*2*1 + 2 + 2) * 2 = 16, P = 9, W = 1.
    tm = oracle_mod.OracleTM(1, 5, 2.0, (4, 4, 1), 2, patch_dim=(2, 2))
    assert (tm.L, tm.W, tm.P) == (16, 1, 9)
    X = np.zeros((1, 16), dtype=np.uint32)
    X[0, 2 * 4 + 1] = 7  # pixel y=2, x=1
    enc = tm.encode(X)
    # patch 4: py = 4 // 3 = 1, px = 4 % 3 = 1.  y-thermometer bit 0; x-thermometer at
    # (DIM1-PD1)+0 = 2; the pixel is (ry, rx) = (1, 0) -> literal 2+2 + 1*2 + 0 = 6.
    pos = [0, 2, 6]
    neg = [8 + l for l in range(8) if l not in pos]
    np.testing.assert_array_equal(enc[0, 4], bits_to_words(pos + neg, 1))
    # patch 0: no thermometer bits, pixel (2,1) outside the patch -> only negations.
    np.testing.assert_array_equal(enc[0, 0], bits_to_words(list(range(8, 16)), 1))
    # patch 8: py = px = 2: y-therm bits 0,1; x-therm bits 2,3; pixel (2,1) outside (x < 2).
    np.testing.assert_array_equal(enc[0, 8], bits_to_words([0, 1, 2, 3] + [12, 13, 14, 15], 1))


def test_encode_vanilla_and_invariants(oracle_mod):
    tm = oracle_mod.OracleTM(1, 5, 2.0, (28, 28, 1), 10)
    assert (tm.L, tm.W, tm.P) == (1568, 49, 1)
    rng = np.random.default_rng(0)
    X = rng.integers(0, 2, (5, 784)).astype(np.uint32)
    enc = tm.encode(X)
    for e in range(5):
        bits = np.unpackbits(enc[e, 0].view(np.uint8), bitorder="little")
        np.testing.assert_array_equal(bits[:784], X[e])          # positive literal = pixel
        np.testing.assert_array_equal(bits[784:1568], 1 - X[e])  # negated half
        assert bits[1568:].sum() == 0                            # beyond L: zero


def test_encode_thermometer_closed_form(oracle_mod):
    # 28x28 with 10x10 patches: ty = tx = 18, P = 361, L = (100 + 36) * 2 = 272.
    tm = oracle_mod.OracleTM(1, 5, 2.0, (28, 28, 1), 10, patch_dim=(10, 10))
    assert (tm.L, tm.W, tm.P) == (272, 9, 361)
    enc = tm.encode(np.zeros((1, 784), dtype=np.uint32))
    for p in (0, 1, 18, 19, 200, 360):
        py, px = divmod(p, 19)
        bits = np.unpackbits(enc[0, p].view(np.uint8), bitorder="little")
        expect = np.zeros(136, dtype=np.uint8)
        expect[:py] = 1
        expect[18:18 + px] = 1
        np.testing.assert_array_equal(bits[:136], expect)
        np.testing.assert_array_equal(bits[136:272], 1 - expect)
        assert bits[272:].sum() == 0


# ------------------------------------------------------------------ inference (kernel.cu:319-394)
def test_score_and_transform_hand_built(oracle_mod):
    tm = oracle_mod.OracleTM(3, 10, 2.0, (4, 1, 1), 2)  # L = 8, P = 1, C = 3
    tm.ta[:] = 0
    tm.ta[0, 0] = 200           # clause 0: x0
    tm.ta[1, [1, 4 + 2]] = 129  # clause 1: x1 AND NOT x2
    # clause 2: empty -> skipped in score, 1 in transform
    tm.w[:] = np.array([[3, -1], [-2, 5], [7, 7]], dtype=np.float32)
    X = np.array([[1, 0, 0, 0], [0, 1, 0, 0], [1, 1, 1, 0], [1, 1, 0, 1]], dtype=np.uint32)
    enc = tm.encode(X)
    cs = tm.score(enc)
    np.testing.assert_array_equal(cs, np.array([[3, -1], [-2, 5], [3, -1], [1, 4]], dtype=np.float32))
    np.testing.assert_array_equal(tm.transform(enc), np.array([[1, 0, 1], [0, 1, 1], [1, 0, 1], [1, 1, 1]]))


def test_score_any_patch(oracle_mod):
    # conv: clause fires if ANY patch matches (early exit over patches).
    tm = oracle_mod.OracleTM(1, 10, 2.0, (3, 1, 1), 2, patch_dim=(1, 1))
    # L = (1 + 2 x-thermometer bits) * 2 = 6, P = 3; include literal 2 (the pixel).
    assert (tm.L, tm.P) == (6, 3)
    tm.ta[:] = 0
    tm.ta[0, 2] = 255
    tm.w[:] = np.array([[2, -3]], dtype=np.float32)
    X = np.array([[0, 0, 0], [0, 0, 1], [1, 1, 1]], dtype=np.uint32)
    enc = tm.encode(X)
    np.testing.assert_array_equal(tm.score(enc), np.array([[0, 0], [2, -3], [2, -3]], dtype=np.float32))
    np.testing.assert_array_equal(tm.transform(enc, True)[:, 0, :], X)


# ------------------------------------------------------------------ training (kernel.cu:285-613)
def block_of(tm):
    return tm.C * tm.P + 2 * tm.C * tm.K + tm.C * tm.K * tm.L


class Inj:
    """Builder of one injected sample block (layout [sel | q | upd | lit])."""

    def __init__(self, tm, fill=0.5):
        self.tm = tm
        self.a = np.full(block_of(tm), fill, dtype=np.float32)

    def sel(self, c, r, u):
        self.a[c * self.tm.P + r - 1] = u

    def q(self, c, k, u):
        self.a[self.tm.C * self.tm.P + c * self.tm.K + k] = u

    def upd(self, c, k, u):
        self.a[self.tm.C * self.tm.P + self.tm.C * self.tm.K + c * self.tm.K + k] = u

    def lit(self, c, k, l, u):
        tm = self.tm
        self.a[tm.C * tm.P + 2 * tm.C * tm.K + (c * tm.K + k) * tm.L + l] = u


def test_type1a_with_s1_and_saturation(oracle_mod):
    # s = 1 (int) -> S_INV = 1.0f: every eligible decrement fires (u <= 1 always).
    tm = oracle_mod.OracleTM(1, 4, 1, (3, 1, 1), 2, init_neg_weights=False)  # L = 6, C = 1, K = 2
    tm.ta[0] = np.array([256, 129, 0, 5, 128, 3], dtype=np.uint32)
    tm.w[0] = [1.0, 1.0]
    X = np.array([[1, 1, 0]], dtype=np.uint32)  # literals: x = 1,1,0 ; negated 0,0,1
    enc = tm.encode(X)
    Y = np.array([[4, -4]], dtype=np.int32)     # class 0 true, class 1 false
    inj = Inj(tm)
    inj.sel(0, 1, 0.1)                          # the only patch is selected
    # class sum: includes are literal 0 (256) and 1 (129): x0 = x1 = 1 -> clause fires.
    # cs = [1, 1]; class 0: v=1, y=4 -> target +1, prob = (4-1)/8 = 0.375.
    inj.upd(0, 0, 0.375)                        # u <= prob -> update
    # class 1: v=1 > -4 -> target -1; Q_PROB = 1.0 (K=2) never skips; prob = (-4-1)/-8 = 0.625
    inj.upd(0, 1, 0.9)                          # no update for class 1
    tm.fit_encoded(enc, Y, inject=inj.a)
    # class 0, sign +1, target +1, fires, n_inc=2 <= L -> Type Ia:
    #   bit 1 literals (0,1,5): +1 below 256 -> 256 (saturated), 130, 4
    #   bit 0 literals (2,3,4): -1 if > 0 -> 0 (stays), 4, 127
    np.testing.assert_array_equal(tm.ta[0], [256, 130, 0, 4, 127, 4])
    np.testing.assert_array_equal(tm.w[0], [2.0, 1.0])
    np.testing.assert_array_equal(tm.pw, [[1]])


def test_type2_increments_once_per_class(oracle_mod):
    # The called type2_fb (kernel.cu:481-506) has no upper guard: two negative classes
    # both giving Type II in one sample add +2 to an excluded 0-literal.
    tm = oracle_mod.OracleTM(1, 4, 2.0, (2, 1, 1), 3, init_neg_weights=False)  # L = 4, K = 3
    tm.ta[0] = np.array([200, 128, 128, 128], dtype=np.uint32)  # clause = x0
    tm.w[0] = [1.0, 1.0, 1.0]
    enc = tm.encode(np.array([[1, 0]], dtype=np.uint32))         # literals 1,0 | 0,1
    Y = np.array([[-4, -4, 4]], dtype=np.int32)                  # classes 0,1 false, 2 true
    inj = Inj(tm)
    inj.sel(0, 1, 0.5)
    # cs = [1,1,1]. Q_PROB = 1.0/2 = 0.5 (q = 1.0 float, K = 3).
    inj.q(0, 0, 0.5)   # 0.5 > 0.5 is false -> not skipped
    inj.q(0, 1, 0.25)
    inj.upd(0, 0, 0.1)  # prob = (-4-1)/-8 = 0.625 -> update
    inj.upd(0, 1, 0.1)
    inj.upd(0, 2, 0.9)  # true class: prob 0.375 -> no update
    tm.fit_encoded(enc, Y, inject=inj.a)
    # Classes 0 and 1: target -1, sign +1 -> Type II twice: 0-literals (1 and 2) get +2.
    np.testing.assert_array_equal(tm.ta[0], [200, 130, 130, 128])
    np.testing.assert_array_equal(tm.w[0], [0.0, 0.0, 1.0])


def test_q_skip_and_positive_polarity_clamp(oracle_mod):
    tm = oracle_mod.OracleTM(1, 4, 2.0, (2, 1, 1), 3, negative_polarity=False, init_neg_weights=False)
    tm.ta[0] = np.array([200, 128, 128, 128], dtype=np.uint32)
    tm.w[0] = [1.0, 1.0, 1.0]
    enc = tm.encode(np.array([[1, 0]], dtype=np.uint32))
    Y = np.array([[-4, -4, 4]], dtype=np.int32)
    inj = Inj(tm)
    inj.sel(0, 1, 0.5)
    inj.q(0, 0, 0.75)   # > Q_PROB 0.5 -> class 0 skipped (no update draw consumed)
    inj.q(0, 1, 0.25)
    inj.upd(0, 0, 0.0)
    inj.upd(0, 1, 0.1)
    inj.upd(0, 2, 0.9)
    tm.fit_encoded(enc, Y, inject=inj.a)
    # Class 1 Type II: w 1 -> 0, clamped to 1 (negative_polarity=False, kernel.cu:603-606).
    np.testing.assert_array_equal(tm.w[0], [1.0, 1.0, 1.0])
    np.testing.assert_array_equal(tm.ta[0], [200, 129, 129, 128])


def test_type1b_when_not_firing(oracle_mod):
    tm = oracle_mod.OracleTM(1, 4, 2.0, (2, 1, 1), 2, init_neg_weights=False)  # S_INV = 0.5 (double)
    tm.ta[0] = np.array([200, 0, 7, 9], dtype=np.uint32)   # clause = x0
    tm.w[0] = [1.0, 1.0]
    enc = tm.encode(np.array([[0, 1]], dtype=np.uint32))   # x0 = 0 -> clause does not fire
    Y = np.array([[4, -4]], dtype=np.int32)
    inj = Inj(tm)
    inj.upd(0, 0, 0.1)   # class 0: cs = 0, prob = 0.5 -> update; target +1, sign +1, not firing -> Ib
    inj.upd(0, 1, 0.9)   # class 1: target -1 (0 > -4), prob 0.5 -> no update
    inj.lit(0, 0, 0, 0.5)   # <= 0.5 -> decrement
    inj.lit(0, 0, 1, 0.1)   # state 0 -> no decrement
    inj.lit(0, 0, 2, 0.51)  # > 0.5 -> keep
    inj.lit(0, 0, 3, 0.2)
    tm.fit_encoded(enc, Y, inject=inj.a)
    np.testing.assert_array_equal(tm.ta[0], [199, 0, 7, 8])
    np.testing.assert_array_equal(tm.w[0], [1.0, 1.0])  # Type Ib leaves the weight
    assert tm.pw.sum() == 0


def test_reservoir_selection(oracle_mod):
    # 3 patches all firing (empty clause fires in training, kernel.cu:273-275).
    tm = oracle_mod.OracleTM(1, 4, 2.0, (3, 1, 1), 2, patch_dim=(1, 1))
    enc = tm.encode(np.array([[1, 0, 1]], dtype=np.uint32))
    Y = np.array([[4, -4]], dtype=np.int32)
    inj = Inj(tm, fill=0.99)
    inj.sel(0, 1, 0.5)   # rank 1: 0.5 < 1     -> patch 0
    inj.sel(0, 2, 0.9)   # rank 2: 0.9 < 0.5?  no
    inj.sel(0, 3, 0.2)   # rank 3: 0.2 < 1/3   -> patch 2
    tm.fit_encoded(enc, Y, inject=inj.a)
    np.testing.assert_array_equal(tm.pw, [[0, 0, 1]])
    # u = 1.0 rejects even rank 1 (strict <, kernel.cu:298): no selection, no vote.
    inj = Inj(tm, fill=0.99)
    for r in (1, 2, 3):
        inj.sel(0, r, 1.0)
    tm.fit_encoded(enc, Y, inject=inj.a)
    np.testing.assert_array_equal(tm.pw, [[0, 0, 1]])
    inj = Inj(tm, fill=0.99)
    inj.sel(0, 1, 0.999)
    inj.sel(0, 2, 0.4999)   # < 0.5 -> patch 1
    inj.sel(0, 3, 1 / 3)    # float(1/3) is not < 1.0f/3 -> keep patch 1
    tm.fit_encoded(enc, Y, inject=inj.a)
    np.testing.assert_array_equal(tm.pw, [[0, 1, 1]])


def test_drop_mask(oracle_mod):
    tm = oracle_mod.OracleTM(2, 4, 2.0, (3, 1, 1), 2)
    enc = tm.encode(np.array([[1, 0, 1]] * 4, dtype=np.uint32))
    Y = np.array([[4, -4]] * 4, dtype=np.int32)
    before_ta, before_w = tm.ta.copy(), tm.w.copy()
    tm.fit_encoded(enc, Y, drop=np.array([1, 1], dtype=np.uint32))
    np.testing.assert_array_equal(tm.ta, before_ta)
    np.testing.assert_array_equal(tm.w, before_w)
    assert tm.pw.sum() == 0


def test_state_bounds_invariant(oracle_mod):
    """0 <= state <= max(256, 128 + K); weights stay integers and move by <= 1 per
    (clause, class) per sample."""
    tm = oracle_mod.OracleTM(8, 5, 2.0, (6, 1, 1), 4)
    rng = np.random.default_rng(9)
    X = rng.integers(0, 2, (300, 6)).astype(np.uint32)
    enc = tm.encode(X)
    Y = tm.encode_y_multiclass(rng.integers(0, 4, 300))
    for i in range(0, 300, 50):
        w0 = tm.w.copy()
        tm.fit_encoded(enc[i:i + 1], Y[i:i + 1])
        assert np.abs(tm.w - w0).max() <= 1
    assert tm.ta.max() <= max(256, 128 + 4)
    assert np.all(tm.w == np.round(tm.w))


def test_clause_banks(oracle_mod):
    """coalesced=False: clause c votes for and learns only its bank's class c // per_bank
    (kernel.cu:306-312 in select_active, :563-565 in clause_update); inference still sums
    every class's weight of a firing clause (kernel.cu:337-339); the initial weights are
    +1 / -1 in the first / second half of the own bank and 0 elsewhere (kernel.cu:58-66)."""
    # 2 clauses per bank, 2 classes -> C = 4; dim (2,1,1): L = 4 (x0, x1, not x0, not x1).
    tm = oracle_mod.OracleTM(2, 4, 2.0, (2, 1, 1), 2, coalesced=False)
    assert tm.C == 4
    np.testing.assert_array_equal(tm.w, [[1, 0], [-1, 0], [0, 1], [0, -1]])
    tm.ta[:] = 128
    tm.ta[0, 0] = 200  # clause 0 (bank 0): x0
    tm.ta[1, 2] = 200  # clause 1 (bank 0): not x0
    tm.ta[2, 0] = 200  # clause 2 (bank 1): x0
    tm.ta[3, 1] = 200  # clause 3 (bank 1): x1
    # out-of-bank weights set non-zero, so that a vote or an update outside the bank shows
    tm.w[:] = np.array([[3, 5], [-1, 0], [-7, 2], [0, -1]], dtype=np.float32)
    enc = tm.encode(np.array([[1, 0]], dtype=np.uint32))  # literals 1, 0, 0, 1
    Y = np.array([[4, -4]], dtype=np.int32)
    inj = Inj(tm, fill=0.0)  # every unset draw would take any branch it is asked for
    for c in range(4):
        inj.sel(c, 1, 0.5)
    # clauses 0 and 2 fire.  Class sums over the own bank only: class 0 = w[0,0] = 3,
    # class 1 = w[2,1] = 2 (not 3 - 7 and 5 + 2).
    # class 0: v = 3 <= 4 -> target +1, prob (4 - 3) / 8 = 0.125;
    # class 1: v = 2 > -4 -> target -1, prob (-4 - 2) / -8 = 0.75; Q_PROB = 1.0 (K = 2).
    inj.upd(0, 0, 0.125)          # clause 0, class 0: u <= prob; sign +1, fires -> Type Ia
    inj.lit(0, 0, 1, 0.5)         #   0-literal x1: 128 -> 127 (u <= S_INV 0.5)
    inj.lit(0, 0, 2, 0.75)        #   0-literal not x0: kept
    inj.upd(1, 0, 0.1)            # clause 1, class 0: sign -1, target +1, not firing -> no branch
    inj.q(2, 1, 0.9)              # clause 2, class 1: not skipped (0.9 <= 1.0)
    inj.upd(2, 1, 0.75)           #   u <= 0.75; sign +1, target -1, fires -> Type II
    inj.q(3, 1, 1.0)              # clause 3, class 1: not skipped (1.0 is not > 1.0)
    inj.upd(3, 1, 0.7)            #   sign -1, target -1, not firing -> Type Ib
    inj.lit(3, 1, 0, 0.5)         #   128 -> 127
    inj.lit(3, 1, 1, 0.6)         #   200 kept
    inj.lit(3, 1, 2, 0.1)         #   128 -> 127
    inj.lit(3, 1, 3, 0.7)         #   128 kept
    upd = tm.fit_encoded(enc, Y, inject=inj.a)
    assert upd == 3 and tm.last_feedback_samples == 1
    np.testing.assert_array_equal(tm.ta[0], [201, 127, 128, 129])  # Ia: 1-literals +1
    np.testing.assert_array_equal(tm.ta[1], [128, 128, 200, 128])
    np.testing.assert_array_equal(tm.ta[2], [200, 129, 129, 128])  # II: 0-literals +1
    np.testing.assert_array_equal(tm.ta[3], [127, 200, 127, 128])
    np.testing.assert_array_equal(tm.w, [[4, 5], [-1, 0], [-7, 1], [0, -1]])
    np.testing.assert_array_equal(tm.pw, [[1], [0], [1], [0]])
    # inference: every class sums a firing non-empty clause's weights (kernel.cu:337-339).
    # The clauses are now 0: x0 AND not x1 (state 129 > 128), 1: not x0, 2: x0 AND x1 AND
    # not x0 (never fires), 3: x1.  (1, 0) fires clause 0 only, and its out-of-bank weight
    # 5 counts for class 1; (0, 1) fires clauses 1 and 3; (0, 0) fires clause 1.
    enc2 = tm.encode(np.array([[1, 0], [0, 1], [0, 0]], dtype=np.uint32))
    np.testing.assert_array_equal(tm.score(enc2), [[4, 5], [-1 + 0, 0 - 1], [-1, 0]])


def test_max_included_literals(oracle_mod):
    """A firing clause with more included literals than MAX_INCLUDED_LITERALS takes Type Ib
    instead of Type Ia (kernel.cu:583-586); at the limit it still takes Type Ia."""
    tm = oracle_mod.OracleTM(2, 4, 2.0, (3, 1, 1), 2, max_included_literals=1, init_neg_weights=False)
    assert tm.C == 2 and tm.L == 6
    tm.ta[:] = 128
    tm.ta[0, [0, 1]] = 150   # clause 0: x0 AND x1 (2 includes > 1)
    tm.ta[1, 0] = 150        # clause 1: x0 (1 include, at the limit)
    tm.w[:] = 1.0
    enc = tm.encode(np.array([[1, 1, 0]], dtype=np.uint32))  # literals 1,1,0 | 0,0,1
    Y = np.array([[4, -4]], dtype=np.int32)
    inj = Inj(tm, fill=0.75)
    inj.sel(0, 1, 0.5)
    inj.sel(1, 1, 0.5)
    # class sums 2 and 2.  Class 0: target +1, prob (4 - 2) / 8 = 0.25.
    # Class 1: target -1, prob (-4 - 2) / -8 = 0.75; u = 0.75 > 0.25 in class 0 by default.
    inj.upd(0, 0, 0.25)
    inj.upd(1, 0, 0.25)
    inj.q(0, 1, 0.5)
    inj.q(1, 1, 0.5)
    inj.upd(0, 1, 0.9)       # class 1: no update for either clause
    inj.upd(1, 1, 0.9)
    for l in range(6):       # literal draws: decrement exactly literals 0, 2, 4
        inj.lit(0, 0, l, 0.5 if l % 2 == 0 else 0.6)
        inj.lit(1, 0, l, 0.5 if l % 2 == 0 else 0.6)
    upd = tm.fit_encoded(enc, Y, inject=inj.a)
    assert upd == 2
    # clause 0, Type Ib: every literal with u <= 0.5 and state > 0 decrements; no weight change
    np.testing.assert_array_equal(tm.ta[0], [149, 150, 127, 128, 127, 128])
    # clause 1, Type Ia: 1-literals (0, 1, 5) +1; 0-literals (2, 3, 4) -1 when u <= 0.5
    np.testing.assert_array_equal(tm.ta[1], [151, 129, 127, 128, 127, 129])
    np.testing.assert_array_equal(tm.w, [[1, 1], [2, 1]])


def test_feedback_sample_count(oracle_mod):
    """A sample counts as a feedback sample when some class's update probability is above
    zero: clipped sums at +T for the true class and -T for the others give none."""
    tm = oracle_mod.OracleTM(1, 1, 2.0, (2, 1, 1), 2, init_neg_weights=False)  # w = [1, 1]
    tm.w[0] = [1.0, -1.0]
    enc = tm.encode(np.array([[1, 0]] * 3, dtype=np.uint32))  # the empty clause fires
    inj = np.full(3 * (tm.C * tm.P + 2 * tm.C * tm.K + tm.C * tm.K * tm.L), 0.5, dtype=np.float32)
    # class sums (1, -1) with T = 1: at the targets (1, -1) -> no feedback; targets (-1, 1)
    # -> both classes have probability 1; (1, 1) -> class 1 has probability 1
    Y = np.array([[1, -1], [-1, 1], [1, 1]], dtype=np.int32)
    # the first sample changes nothing, so the later ones see the same sums
    tm.fit_encoded(enc[:1], Y[:1], inject=inj[:inj.size // 3])
    assert tm.last_feedback_samples == 0
    tm.fit_encoded(enc[1:2], Y[1:2], inject=np.full(inj.size // 3, 1.0, dtype=np.float32))
    assert tm.last_feedback_samples == 1
