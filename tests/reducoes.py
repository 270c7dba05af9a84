"""Inputs on which a head-width-64 attention problem reduces exactly to a head-width-4 one, and the maps between
their outputs. They pin the generalized attention (the declared extension of ops.py:186-258 used at config 4 and
5) to the spec's own head-width-4 code, which the reference's goldens pin.

Construction, at BLK = 32, T <= 128, Bt sequences:
  * the head-width-4 problem: D4 = 256, H4 = 64 heads (the spec's shape), any inputs;
  * the head-width-64 problem: D64 = 512, H64 = 8 heads. Head h carries head 8h of the head-width-4 problem in
    its first 4 dimensions with the exponent of the block that holds them (a block of 32 columns holds heads
    8h .. 8h + 7 there); its other 60 dimensions are 0, and its second block of 32 columns is an all-zero block
    (exponent -127), so the head's alignment maximum is the first block's over the tokens, as for head 8h.
    Head h of 8 gets ALiBi slope 8 - (8 h) / 8 = 8 - h; head 8h of 64 gets the spec's 8 - 8h // 8: the same.
  * the score shift is -(eq + ek - log2(hd)/2 + 8): -1 + ... at head width 4, -3 + ... at 64. The q block
    exponents of the head-width-64 problem are the head-width-4 ones + 2, so both shifts are equal, and with them
    u, P and o (and in the backward every maximum, shift and product).
Outputs then match: P64[b, h] = P4[b, 8h]; o64[:, 64h + d] = o4[:, 32h + d] for d < 4 and 0 for d >= 4, with equal
exponents; the backward's gq, gv equal on those columns, and gk equal with its exponent 2 larger (eq is 2 larger).
"""
import numpy as np

import recipe as R

BLK = 32
D4, H4, D64, H64 = 256, 64, 512, 8
E_ZERO = -127


def problemas(semente, Bt, T):
    """((qkv4 m, E), (go4 m, E)) and ((qkv64 m, E), (go64 m, E)) as numpy arrays."""
    M = Bt * T
    qm4, qE4 = R.bloco(R.substream(semente, "qkv4"), M, 3 * D4, BLK, espalha=4, e0=-6, zera=0.05)
    gm4, gE4 = R.bloco(R.substream(semente, "go4"), M, D4, BLK, espalha=5, e0=-20, zera=0.05)
    qm64 = np.zeros((M, 3 * D64), np.int8)
    qE64 = np.full((M, 3 * D64 // BLK), E_ZERO, np.int8)
    gm64 = np.zeros((M, D64), np.int8)
    gE64 = np.full((M, D64 // BLK), E_ZERO, np.int8)
    for h in range(H64):
        for part in range(3):              # q, k, v
            c4, c64 = part * D4 + 32 * h, part * D64 + 64 * h
            qm64[:, c64:c64 + 4] = qm4[:, c4:c4 + 4]
            e = qE4[:, c4 // BLK].astype(np.int64)
            if part == 0:                  # q: exponent + 2, except on zero blocks
                e = np.where(e == E_ZERO, E_ZERO, e + 2)
            qE64[:, c64 // BLK] = e.astype(np.int8)
        gm64[:, 64 * h:64 * h + 4] = gm4[:, 32 * h:32 * h + 4]
        gE64[:, 2 * h] = gE4[:, h]
    return ((qm4, qE4), (gm4, gE4)), ((qm64, qE64), (gm64, gE64))


def confere_frente(saida4, saida64, Bt):
    """Asserts the forward outputs ((oacc, oe), P) of the two problems match as the module docstring states."""
    (o4, e4), P4 = (np.asarray(x) for x in saida4[0]), np.asarray(saida4[1])
    (o64, e64), P64 = (np.asarray(x) for x in saida64[0]), np.asarray(saida64[1])
    T = P4.shape[-1]
    P4 = P4.reshape(Bt, H4, T, T)
    P64 = P64.reshape(Bt, H64, T, T)
    for h in range(H64):
        assert np.array_equal(P64[:, h], P4[:, 8 * h]), f"P of head {h}"
        assert np.array_equal(o64[:, 64 * h:64 * h + 4], o4[:, 32 * h:32 * h + 4]), f"o of head {h}"
        assert not np.any(o64[:, 64 * h + 4:64 * h + 64]), f"o of head {h}: the zero dimensions"
        assert np.array_equal(e64[:, 64 * h:64 * h + 4], e4[:, 32 * h:32 * h + 4]), f"o exponents of head {h}"


def confere_tras(g4, g64):
    """Asserts the backward raw outputs (acc, e) [M, 3D] of the two problems match (gk's exponent + 2)."""
    a4, e4 = (np.asarray(x).astype(np.int64) for x in g4)
    a64, e64 = (np.asarray(x).astype(np.int64) for x in g64)
    for h in range(H64):
        for part, nome, de in ((0, "gq", 0), (1, "gk", 2), (2, "gv", 0)):
            c4, c64 = part * D4 + 32 * h, part * D64 + 64 * h
            assert np.array_equal(a64[:, c64:c64 + 4], a4[:, c4:c4 + 4]), f"{nome} of head {h}"
            assert np.array_equal(e64[:, c64:c64 + 4], e4[:, c4:c4 + 4] + de), f"{nome} exponents of head {h}"
            assert not np.any(a64[:, c64 + 4:c64 + 64]), f"{nome} of head {h}: the zero dimensions"
