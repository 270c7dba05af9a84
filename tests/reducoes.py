"""Inputs on which the head-width-64 attention (the declared extension of ops.py:186-258 used at configs 4 and 5)
has a known answer, and the maps between outputs. Three families, each chosen so that a plausible mistake in a
head's dimensions 4..63 or in its second block of 32 columns changes bits:

1. Reduction to the spec's head width 4 (`problemas`, `confere_frente`, `confere_tras`), at BLK = 32, T <= 128:
  * the head-width-4 problem: D4 = 256, H4 = 64 heads (the spec's shape), any inputs;
  * the head-width-64 problem: D64 = 512, H64 = 8 heads. Head h carries head 8h of the head-width-4 problem in
    its dimensions `desloc` .. `desloc` + 3 with the exponent of the block that holds them (a block of 32 columns
    holds heads 8h .. 8h + 7 there); its other 60 dimensions are 0, and its other block of 32 columns is an
    all-zero block (exponent -127), so the head's alignment maximum is the loaded block's over the tokens, as
    for head 8h. With `desloc` >= 32 the data sits in the head's second block and the first block is the zero one.
    Head h of 8 gets ALiBi slope 8 - (8 h) / 8 = 8 - h; head 8h of 64 gets the spec's 8 - 8h // 8: the same.
  * the score shift is -(eq + ek - log2(hd)/2 + 8): -1 + ... at head width 4, -3 + ... at 64. The q block
    exponents of the head-width-64 problem are the head-width-4 ones + 2, so both shifts are equal, and with them
    u, P and o (and in the backward every maximum, shift and product).
  Outputs then match: P64[b, h] = P4[b, 8h]; o64[:, 64h + desloc + d] = o4[:, 32h + d] for d < 4 and 0 elsewhere
  in the head, with equal exponents; the backward's gq, gv equal on those columns, and gk equal with its exponent 2
  larger (eq is 2 larger).

2. v = 0 (`problema_v_zero`): every v block of every head is an all-zero block. Then gP = dO v^T = 0, so both
   shrink counts are 0, s_lin = 0, dS = 0 and gq = gk = 0 exactly, while gv_j = sum_i P_ij a_i over all 64
   dimensions (a: dO aligned to the head's largest block exponent over both blocks and all T tokens, with GA = 4
   guard bits), at exponent emx - GA - 8. q, k and dO are random in every dimension of both blocks.

3. Head-dimension permutation (`problema_permutado`): per token and head, both blocks of q carry one exponent (and
   so for k, v and dO). Alignment then treats every dimension of a head alike, the score q.k is invariant under a
   joint permutation of the q and k dimensions, and dO.v under a joint permutation of the v and dO dimensions.
   So permuting q, k by pi and v, dO by sigma (per head, across both blocks) leaves P unchanged and permutes o and
   gv by sigma and gq, gk by pi, bit for bit, in both backward variants.
"""
import numpy as np

import recipe as R

BLK = 32
D4, H4, D64, H64 = 256, 64, 512, 8
HD = D64 // H64
GA = 4
E_ZERO = -127


def problemas(semente, Bt, T, desloc=0):
    """((qkv4 m, E), (go4 m, E)) and ((qkv64 m, E), (go64 m, E)) as numpy arrays; `desloc` (a multiple of 4,
    0 .. 60) is where head 8h's 4 dimensions sit inside head h of the head-width-64 problem."""
    assert desloc % 4 == 0 and 0 <= desloc <= HD - 4
    M = Bt * T
    qm4, qE4 = R.bloco(R.substream(semente, "qkv4"), M, 3 * D4, BLK, espalha=4, e0=-6, zera=0.05)
    gm4, gE4 = R.bloco(R.substream(semente, "go4"), M, D4, BLK, espalha=5, e0=-20, zera=0.05)
    qm64 = np.zeros((M, 3 * D64), np.int8)
    qE64 = np.full((M, 3 * D64 // BLK), E_ZERO, np.int8)
    gm64 = np.zeros((M, D64), np.int8)
    gE64 = np.full((M, D64 // BLK), E_ZERO, np.int8)
    for h in range(H64):
        for part in range(3):              # q, k, v
            c4, c64 = part * D4 + 32 * h, part * D64 + HD * h + desloc
            qm64[:, c64:c64 + 4] = qm4[:, c4:c4 + 4]
            e = qE4[:, c4 // BLK].astype(np.int64)
            if part == 0:                  # q: exponent + 2, except on zero blocks
                e = np.where(e == E_ZERO, E_ZERO, e + 2)
            qE64[:, c64 // BLK] = e.astype(np.int8)
        c64 = HD * h + desloc
        gm64[:, c64:c64 + 4] = gm4[:, 32 * h:32 * h + 4]
        gE64[:, c64 // BLK] = gE4[:, h]
    return ((qm4, qE4), (gm4, gE4)), ((qm64, qE64), (gm64, gE64))


def confere_frente(saida4, saida64, Bt, desloc=0):
    """Asserts the forward outputs ((oacc, oe), P) of the two problems match as family 1 states."""
    (o4, e4), P4 = (np.asarray(x) for x in saida4[0]), np.asarray(saida4[1])
    (o64, e64), P64 = (np.asarray(x) for x in saida64[0]), np.asarray(saida64[1])
    T = P4.shape[-1]
    P4 = P4.reshape(Bt, H4, T, T)
    P64 = P64.reshape(Bt, H64, T, T)
    for h in range(H64):
        c = HD * h + desloc
        outros = np.r_[HD * h:c, c + 4:HD * (h + 1)]
        assert np.array_equal(P64[:, h], P4[:, 8 * h]), f"P of head {h}"
        assert np.array_equal(o64[:, c:c + 4], o4[:, 32 * h:32 * h + 4]), f"o of head {h}"
        assert not np.any(o64[:, outros]), f"o of head {h}: the zero dimensions"
        assert np.array_equal(e64[:, c:c + 4], e4[:, 32 * h:32 * h + 4]), f"o exponents of head {h}"


def confere_tras(g4, g64, desloc=0):
    """Asserts the backward raw outputs (acc, e) [M, 3D] of the two problems match (gk's exponent + 2)."""
    a4, e4 = (np.asarray(x).astype(np.int64) for x in g4)
    a64, e64 = (np.asarray(x).astype(np.int64) for x in g64)
    for h in range(H64):
        for part, nome, de in ((0, "gq", 0), (1, "gk", 2), (2, "gv", 0)):
            c4, c64 = part * D4 + 32 * h, part * D64 + HD * h + desloc
            outros = np.r_[part * D64 + HD * h:c64, c64 + 4:part * D64 + HD * (h + 1)]
            assert np.array_equal(a64[:, c64:c64 + 4], a4[:, c4:c4 + 4]), f"{nome} of head {h}"
            assert np.array_equal(e64[:, c64:c64 + 4], e4[:, c4:c4 + 4] + de), f"{nome} exponents of head {h}"
            assert not np.any(a64[:, outros]), f"{nome} of head {h}: the zero dimensions"


def problema_v_zero(semente, Bt, T):
    """Family 2: ((qkv m, E), (go m, E)) at D = 512, H = 8, BLK = 32, with every v block all-zero (E = -127) and
    q, k, dO random in every block, exponents spread over a few steps so that a head's two blocks differ."""
    M = Bt * T
    qm, qE = R.bloco(R.substream(semente, "qkv"), M, 3 * D64, BLK, espalha=3, e0=-7, zera=0.03)
    gm, gE = R.bloco(R.substream(semente, "go"), M, D64, BLK, espalha=6, e0=-20, zera=0.03)
    qm[:, 2 * D64:] = 0
    qE[:, 2 * D64 // BLK:] = E_ZERO
    return (qm, qE), (gm, gE)


def gv_v_zero(go, P, Bt, T):
    """Family 2's closed form: gv (int64 [M, D]) and its exponent per (sequence, head) from dO and P alone.
    Alignment (ops.py:186-192 over the head's two blocks): a = m 2^(E - emx + GA), rounded half to even, emx the
    head's largest block exponent over its T tokens; gv_j = sum_{i >= j} P_ij a_i (P stored [j][i])."""
    gm, gE = (np.asarray(x).astype(np.int64) for x in go)
    P = np.asarray(P).astype(np.int64).reshape(Bt, H64, T, T)      # [b][h][j][i]
    gv = np.zeros((Bt * T, D64), np.int64)
    expo = np.zeros((Bt, H64), np.int64)
    for b in range(Bt):
        for h in range(H64):
            rows = slice(b * T, (b + 1) * T)
            Eb = gE[rows, 2 * h:2 * h + 2]                           # [T, 2]
            emx = int(Eb.max())
            e = np.repeat(Eb, BLK, axis=1) - emx + GA                  # [T, 64]
            a = _rnd_meio_par(gm[rows, HD * h:HD * (h + 1)], e)
            gv[rows, HD * h:HD * (h + 1)] = P[b, h] @ a                # sum_i P[j][i] a_i
            expo[b, h] = emx - GA - 8
    return gv, expo


def _rnd_meio_par(m, e):
    """m 2^e rounded half to even, elementwise (int64 m, e; e >= -62): by exact integer arithmetic."""
    m = m.astype(np.int64)
    e = e.astype(np.int64)
    out = np.where(e >= 0, m << np.maximum(e, 0), 0)
    s = np.minimum(np.maximum(-e, 1), 62)
    q = np.floor_divide(m, np.int64(1) << s)                          # floor(m / 2^s)
    r = m - (q << s)                                                  # 0 <= r < 2^s
    meio = np.int64(1) << (s - 1)
    cima = (r > meio) | ((r == meio) & (q & 1 == 1))
    return np.where(e >= 0, out, q + cima)


def problema_permutado(semente, Bt, T):
    """Family 3: (qkv, go) with one exponent per (token, head) on both blocks of q, k, v and dO, and the same
    problem with every head's q, k dimensions permuted by pi[h] and v, dO dimensions by sigma[h].
    Returns (qkv, go), (qkv_p, go_p), pi [H, 64], sigma [H, 64]; column c of a permuted head holds dimension
    pi[h][c] (or sigma[h][c]) of the original."""
    M = Bt * T
    qm, qE = R.bloco(R.substream(semente, "qkv"), M, 3 * D64, BLK, espalha=3, e0=-7)
    gm, gE = R.bloco(R.substream(semente, "go"), M, D64, BLK, espalha=6, e0=-20)
    qE[:, 1::2] = qE[:, 0::2]                  # block 2h + 1 of each part = block 2h: one exponent per head
    gE[:, 1::2] = gE[:, 0::2]
    chave = lambda tag: R.uniform01(R.substream(semente, tag), (H64, HD))
    pi, sigma = np.argsort(chave("pi"), axis=1), np.argsort(chave("sigma"), axis=1)
    qp, gp = qm.copy(), gm.copy()
    for h in range(H64):
        base = HD * h
        for part, perm in ((0, pi[h]), (1, pi[h]), (2, sigma[h])):
            c = part * D64 + base
            qp[:, c:c + HD] = qm[:, c + perm]
        gp[:, base:base + HD] = gm[:, base + sigma[h]]
    return ((qm, qE), (gm, gE)), ((qp, qE.copy()), (gp, gE.copy())), pi, sigma


def permuta_colunas(x, perms, D, part):
    """x [M, k D] with head h's columns of part `part` permuted by perms[h] (as problema_permutado does)."""
    y = np.array(x, copy=True)
    for h in range(H64):
        c = part * D + HD * h
        y[:, c:c + HD] = x[:, c + perms[h]]
    return y
