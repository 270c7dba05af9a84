"""Pins the CPU oracle (oracle/jatai_oracle.cpp) before anything is compared against it.

Checks, per function:
  * reference golden vectors written from the spec `OpsRef` (tests/golden/*.json, see make_golden.py):
    every op case at BLK 128 and 32, config 1, primitive tables, two full training steps;
  * closed forms that a plausible mistake would break: bitlen = int.bit_length, rnd = exact round-half-even
    (Fraction), isqrt = floor sqrt for n >= 1, the GEMM's equal-exponent case = integer matmul + quant, split
    invariance of the raw GEMM, the R16 round trip.
"""
import json
import math
import os
from fractions import Fraction

import numpy as np
import pytest
import torch

import cases as CS
import recipe as R
from oracle.ops_oracle import OpsOraculo, g_rms

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _gold(nome):
    return json.load(open(os.path.join(GOLD, nome)))


def host(t):
    return t.detach().cpu().numpy()


class BE:
    def __init__(self, blk):
        self.ops = OpsOraculo(blk)

    def dev(self, a):
        return torch.from_numpy(np.ascontiguousarray(a))

    def limite(self, flag):
        old, self.ops.limite = self.ops.limite, flag
        return old


# ---------------------------------------------------------------- primitives
def test_primitives_vs_golden():
    g = _gold("primitives.json")
    d = np.arange(0, 7001, dtype=np.int64)
    assert R.sha(OpsOraculo.prim("exp_int", d)) == g["exp_int"]["sha"]
    n = np.concatenate([np.arange(0, 70000), R.uniform_int(7, (200000,), 0, (1 << 30) - 1)]).astype(np.int64)
    assert R.sha(OpsOraculo.prim("isqrt", n)) == g["isqrt"]["sha"]
    x = R.uniform_int(8, (100000,), -(1 << 29), (1 << 29) - 1)
    s = R.uniform_int(9, (100000,), -8, 40)
    assert R.sha(OpsOraculo.prim("rnd", x, s)) == g["rnd"]["sha"]
    assert R.sha(OpsOraculo.prim("bitlen", x)) == g["bitlen"]["sha"]


def test_primitives_closed_forms():
    x = R.uniform_int(11, (3000,), -(1 << 40), 1 << 40)
    s = R.uniform_int(12, (3000,), -10, 50)
    x[:50] = 0
    bl = OpsOraculo.prim("bitlen", x)
    assert all(int(b) == abs(int(v)).bit_length() for v, b in zip(x, bl))
    x2 = x.copy()
    x2[(s < 0)] = x2[(s < 0)] >> 12                      # left shifts stay in int64
    rn = OpsOraculo.prim("rnd", x2, s)
    for v, sh, r in zip(x2, s, rn):
        v, sh = int(v), int(sh)
        if sh <= 0:
            assert int(r) == v << -sh
            continue
        q = Fraction(v, 1 << sh)
        f = math.floor(q)
        exp = f + 1 if q - f > Fraction(1, 2) else f if q - f < Fraction(1, 2) else (f if f % 2 == 0 else f + 1)
        assert int(r) == exp, (v, sh, int(r), exp)
    n = np.concatenate([np.arange(1, 5000), R.uniform_int(13, (5000,), 1, (1 << 30) - 1)]).astype(np.int64)
    iq = OpsOraculo.prim("isqrt", n)
    assert all(int(q) == math.isqrt(int(v)) for v, q in zip(n, iq))
    # exp_int(0) is 1.0 in Q15 within the polynomial's error; monotone non-increasing over its domain
    ex = OpsOraculo.prim("exp_int", np.arange(0, 7001))
    assert abs(int(ex[0]) - 32768) <= 8 and np.all(np.diff(ex) <= 0) and int(ex[-1]) == 0
    ref = np.exp(-np.arange(0, 6001) / 256.0) * 32768
    assert np.max(np.abs(ex[:6001] - ref)) < 8


def test_g_rms():
    # ops.py:28-30 at BLK 128 (reference shapes) and the values the BLK=32 extension uses
    assert g_rms(256, 128) == (6, 6)
    assert g_rms(512, 32) == (4, 5)


# ---------------------------------------------------------------- op cases vs the reference spec
@pytest.mark.parametrize("blk", [128, 32])
def test_ops_vs_golden(blk):
    gold = _gold(f"ops_blk{blk}.json")
    be = BE(blk)
    casos = CS.casos()
    assert [c["nome"] for c in gold] == [n for n, _ in casos]
    falhas = []
    for i, ((nome, fn), gc) in enumerate(zip(casos, gold)):
        rec = CS.Gravador(be.ops, host)
        g = CS.Gen(R.substream(1000 + i, nome), blk, be.dev)
        fn(rec, g, be)
        if [list(x) for x in rec.log] != [list(x) for x in gc["chamadas"]]:
            falhas.append(nome)
    assert not falhas, f"oracle differs from the spec at BLK={blk}: {falhas}"


@pytest.mark.parametrize("blk", [128, 32])
def test_ops_dominio_vs_golden(blk):
    """The rest of the reference's shape domain (row widths 384-896, softmax V = 384 / 640, head-width-4
    attention at H = 32 and T = 32 / 96) against the spec's own outputs."""
    gold = _gold(f"ops_dominio_blk{blk}.json")
    be = BE(blk)
    casos = CS.casos_dominio()
    assert [c["nome"] for c in gold] == [n for n, _ in casos]
    falhas = []
    for i, ((nome, fn), gc) in enumerate(zip(casos, gold)):
        rec = CS.Gravador(be.ops, host)
        g = CS.Gen(R.substream(1000 + i, nome), blk, be.dev)
        fn(rec, g, be)
        if [list(x) for x in rec.log] != [list(x) for x in gc["chamadas"]]:
            falhas.append(nome)
    assert not falhas, f"oracle differs from the spec at BLK={blk}: {falhas}"


def test_config1_vs_golden():
    gold = _gold("config1.json")
    for blk in (32, 128):
        ops = OpsOraculo(blk)
        A = tuple(torch.from_numpy(x) for x in R.bloco(R.substream(0, "A"), 512, 512, blk, espalha=4, e0=-4))
        B = tuple(torch.from_numpy(x) for x in R.bloco(R.substream(0, "B"), 512, 512, blk, espalha=4, e0=-4))
        assert [R.sha(host(t)) for t in ops.gemm(A, B)] == gold[str(blk)]["bloco"]
        assert [R.sha(host(t)) for t in ops.gemm(A, B, cru=True)] == gold[str(blk)]["cru"]


# ---------------------------------------------------------------- GEMM closed form and invariants
@pytest.mark.parametrize("blk", [32, 128])
def test_gemm_equal_exponents_is_integer_matmul(blk):
    """With every exponent of A's rows and B's rows equal, all alignment shifts are 0 and the raw output is
    16 * (A.B^T) exactly with exponent RA + RB - 4 (the textbook integer matmul)."""
    M, N, K = 64, 96, 4 * blk
    a = R.uniform_int(21, (M, K), -127, 127).astype(np.int8)
    b = R.uniform_int(22, (N, K), -127, 127).astype(np.int8)
    ea = np.full((M, K // blk), -9, np.int8)
    eb = np.full((N, K // blk), -5, np.int8)
    ops = OpsOraculo(blk)
    acc, e = ops.gemm((torch.from_numpy(a), torch.from_numpy(ea)), (torch.from_numpy(b), torch.from_numpy(eb)), cru=True)
    ref = 16 * (a.astype(np.int64) @ b.astype(np.int64).T)
    assert np.array_equal(host(acc).astype(np.int64), ref)
    assert np.all(host(e) == -9 - 5 - 4)


@pytest.mark.parametrize("blk", [32, 128])
def test_gemm_spread_exponents_brute_force(blk):
    """Ragged shapes (M not a multiple of 4, N not of 16) and exponents spread over the whole int8 range, so
    alignment shifts run from 0 to past the mantissa width: each raw output equals the sum over K-blocks of the
    exact rational 16 * dot / 2^shift rounded half to even (Python's round on a Fraction)."""
    M, N, K = 7, 19, 4 * blk
    a = R.uniform_int(41, (M, K), -128, 127).astype(np.int8)
    b = R.uniform_int(42, (N, K), -128, 127).astype(np.int8)
    ea = R.uniform_int(43, (M, K // blk), -127, 60).astype(np.int8)
    eb = R.uniform_int(44, (N, K // blk), -127, 60).astype(np.int8)
    ea[0, :] = -127
    eb[3, 1] = 60
    ops = OpsOraculo(blk)
    acc, e = ops.gemm((torch.from_numpy(a), torch.from_numpy(ea)), (torch.from_numpy(b), torch.from_numpy(eb)), cru=True)
    acc, e = host(acc).astype(np.int64), host(e).astype(np.int64)
    RA, RB = ea.astype(np.int64).max(1), eb.astype(np.int64).max(1)
    for i in range(M):
        for j in range(N):
            s = 0
            for q in range(K // blk):
                p = int(np.dot(a[i, q * blk:(q + 1) * blk].astype(np.int64), b[j, q * blk:(q + 1) * blk].astype(np.int64)))
                sh = int(RA[i] - ea[i, q]) + int(RB[j] - eb[j, q])
                s += round(Fraction(16 * p, 2 ** sh))
            assert acc[i, j] == s, (i, j)
            assert e[i, j] == max(RA[i] + RB[j] - 4, -30000)


def test_gemm_raw_split_invariance():
    """The raw output over K equals the sum of raw outputs over K halves when RA/RB are held fixed: the spec's
    per-block rounding makes the sum over K-blocks associative (the split-K argument)."""
    blk, M, N, K = 32, 32, 48, 256
    A = R.bloco(31, M, K, blk, espalha=6)
    B = R.bloco(32, N, K, blk, espalha=6)
    ops = OpsOraculo(blk)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x))
    full = host(ops.gemm((t(A[0]), t(A[1])), (t(B[0]), t(B[1])), cru=True)[0]).astype(np.int64)
    # pin each half's row maxima to the full-K maxima by appending one all-zero block carrying that maximum
    parts = 0
    for h in range(2):
        sl = slice(h * K // 2, (h + 1) * K // 2)
        bs = slice(h * K // 2 // blk, (h + 1) * K // 2 // blk)
        am = np.concatenate([A[0][:, sl], np.zeros((M, blk), np.int8)], 1)
        ae = np.concatenate([A[1][:, bs], A[1].max(1, keepdims=True)], 1)
        bm = np.concatenate([B[0][:, sl], np.zeros((N, blk), np.int8)], 1)
        be_ = np.concatenate([B[1][:, bs], B[1].max(1, keepdims=True)], 1)
        parts = parts + host(ops.gemm((t(am), t(ae)), (t(bm), t(be_)), cru=True)[0]).astype(np.int64)
    assert np.array_equal(full, parts)


def test_r16_round_trip_and_sum():
    """para8(para16(x)) == x exactly, and soma16 is closer to the exact float64 sum than soma
    (the reference's own check, jatai_cuda/teste_res16.py:27-46)."""
    blk = 128
    ops = OpsOraculo(blk)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x))
    x = tuple(t(v) for v in R.bloco(41, 256, 512, blk, espalha=7, e0=-3))
    back = ops.para8(ops.para16(x))
    deq = lambda m, E: host(m).astype(np.float64) * np.exp2(np.repeat(host(E).astype(np.float64), blk, 1))
    assert np.array_equal(deq(*back), deq(*x))
    y = tuple(t(v) for v in R.bloco(42, 256, 512, blk, espalha=7, e0=-15))
    exato = deq(*x) + deq(*y)
    e16 = np.linalg.norm(deq(*ops.soma16(ops.para16(x), y)) - exato)
    e8 = np.linalg.norm(deq(*ops.soma(x, y)) - exato)
    assert e16 < e8 / 8          # 15-bit vs 7-bit mantissas; measured ratio ~16 at a 2^-12 addend


@pytest.mark.parametrize("blk", [32, 128])
def test_soma_estocastica(blk):
    """gemm_soma's stochastic residual rounding (jt_res_estocastico; no spec, restated from jatai_cuda.cu:146-159
    and :375). Where no bit is dropped it equals the deterministic soma. Over many rows holding the same values
    (each row other seeds) the mean of x + y approaches the exact sum, where half-to-even rounding keeps a fixed
    bias: 100 + 3/256 rounds to 100 every time, and stochastically up with probability 3/256."""
    ops = OpsOraculo(blk)
    NL, C = 4096, 256
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    # no bit dropped: equal exponents and |x + y| <= 127
    x = R.uniform_int(61, (NL, C), -60, 60).astype(np.int8)
    y = R.uniform_int(62, (NL, C), -60, 60).astype(np.int8)
    e = R.uniform_int(63, (NL, C // blk), -20, 5).astype(np.int8)
    X, Y = (t(x), t(e)), (t(y), t(e.copy()))
    assert all(np.array_equal(host(a), host(b)) for a, b in zip(ops.soma_est(X, Y), ops.soma(X, Y)))
    # unbiased where half-to-even is not
    X = (t(np.full((NL, C), 100, np.int8)), t(np.zeros((NL, C // blk), np.int8)))
    Y = (t(np.full((NL, C), 3, np.int8)), t(np.full((NL, C // blk), -8, np.int8)))
    deq = lambda Z: host(Z[0]).astype(np.float64) * np.repeat(2.0 ** host(Z[1]).astype(np.float64), blk, axis=1)
    exato = 100 + 3 / 256
    assert np.all(deq(ops.soma(X, Y)) == 100.0)
    media = deq(ops.soma_est(X, Y)).mean()
    assert abs(media - exato) < 0.002, media


def test_ops_conferido_aponta_divergencia(tmp_path):
    """OpsConferido (the reference's checked wrapper, ops.py:519-560) over a CPU backend: agreement passes the
    backend's outputs through; a backend whose soma is off by one in a single mantissa fails with the op, the
    output and the first differing index. The planted mistake lives in this CPU stand-in, not in any GPU code."""
    from jatai_amd import ops as O
    from jatai_amd.registro import ErroJatai, Registro
    from oracle.ops_oracle import OpsConferido
    O.BLK = 32
    try:
        reg = Registro(str(tmp_path), "conferido", eco=False)
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a))
        X = (t(R.uniform_int(71, (64, 128), -100, 100).astype(np.int8)), t(R.uniform_int(72, (64, 4), -10, 5).astype(np.int8)))
        Y = (t(R.uniform_int(73, (64, 128), -100, 100).astype(np.int8)), t(R.uniform_int(74, (64, 4), -10, 5).astype(np.int8)))
        ok = OpsConferido(reg, OpsOraculo(32))
        Z = ok.soma(X, Y)
        assert np.array_equal(host(Z[0]), host(OpsOraculo(32).soma(X, Y)[0])) and ok.n == {"soma": 1}

        class Torto(OpsOraculo):
            def soma(self, A, B):
                m, e = super().soma(A, B)
                m = m.clone()
                m[3, 17] += 1 if m[3, 17] < 127 else -1
                return m, e
        with pytest.raises(ErroJatai, match=r"conferencia 'soma' / mantissa/acc: 1 de 8192 valores[\s\S]*primeiro em \[3, 17\]"):
            OpsConferido(reg, Torto(32)).soma(X, Y)
    finally:
        O.BLK = 128


# ---------------------------------------------------------------- pins of the functions without a spec
def test_hash32_e_lowbias32():
    """The stochastic rounding's hash (jatai_cuda.cu:146-149) is Wellons' lowbias32: two xorshift-multiply rounds
    with 0x7feb352d and 0x846ca68b. Checked through its published inverse (xorshifts undone, the multipliers'
    inverses mod 2^32: 0x43021123 and 0x1d69e2a5), which must return every input, and the multipliers'
    inverses are checked as such."""
    assert (0x846CA68B * 0x43021123) % (1 << 32) == 1 and (0x7FEB352D * 0x1D69E2A5) % (1 << 32) == 1
    x = np.concatenate([np.arange(0, 4096), R.uniform_int(17, (20000,), 0, (1 << 32) - 1)]).astype(np.int64)
    h = OpsOraculo.prim("hash32", x).astype(np.uint64)
    M = np.uint64(0xFFFFFFFF)
    y = h ^ (h >> np.uint64(16))
    y = (y * np.uint64(0x43021123)) & M
    y = y ^ (y >> np.uint64(15)) ^ (y >> np.uint64(30))
    y = (y * np.uint64(0x1D69E2A5)) & M
    y = y ^ (y >> np.uint64(16))
    assert np.array_equal(y.astype(np.int64), x)
    assert len(np.unique(h)) == len(np.unique(x))          # a bijection
    assert int(OpsOraculo.prim("hash32", np.array([0]))[0]) == 0


def _quant_exata(V, S, mbits, lim, blk):
    """Block quantization of exact dyadic values V_k 2^S_k (Python ints), the spec's rules (ops.py:58-72) on exact
    values: topo = max(S + bitlen(V)), E = topo - mbits, q = round half even (V 2^(S - E)), E + 1 if some |q| > lim,
    zero block if all V are 0 or E < -126. Returns (mantissas, E) per block."""
    def rhe(v, s):                                         # v 2^-s rounded half to even (s may be <= 0)
        if s <= 0:
            return v << -s
        q, r = divmod(v, 1 << s)
        meio = 1 << (s - 1)
        return q + (1 if r > meio or (r == meio and q & 1) else 0)
    ms, Es = [], []
    for b in range(0, len(V), blk):
        vb, sb = V[b:b + blk], S[b:b + blk]
        topos = [s + abs(v).bit_length() for v, s in zip(vb, sb) if v]
        if not topos:
            ms += [0] * blk; Es.append(E_ZERO_)
            continue
        E = max(topos) - mbits
        q = [rhe(v, E - s) for v, s in zip(vb, sb)]
        if any(abs(x) > lim for x in q):
            E += 1
            q = [rhe(v, E - s) for v, s in zip(vb, sb)]
        if E < -126:
            ms += [0] * blk; Es.append(E_ZERO_)
            continue
        ms += [max(-lim, min(lim, x)) for x in q]
        Es.append(E)
    return ms, Es


E_ZERO_ = -127


@pytest.mark.parametrize("blk", [32, 128])
def test_r16_formas_fechadas(blk):
    """The 16-bit residual trio (no spec; jatai_cuda.cu:446-531) against closed forms on exact values:
    para16 is exact (m << 7, E - 7; zero blocks stay zero blocks); para8 is the INT8 block quantization of the
    exact R16 value; soma16 is the 15-bit block quantization (|m| <= 32767) of the exact sum x + y, rounded once --
    its alignment to ec = max(ex + 15, ey + 7) - 28 loses nothing that the final rounding keeps. Exponent gaps from
    -30 to +30 between x and y, and zero blocks on either side."""
    ops = OpsOraculo(blk)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    Rn, C = 64, 4 * blk
    x8 = R.bloco(91, Rn, C, blk, espalha=6, e0=-3, zera=0.1)
    p16 = ops.para16(tuple(t(v) for v in x8))
    m16, E16 = host(p16[0]).astype(np.int64), host(p16[1]).astype(np.int64)
    assert np.array_equal(m16, x8[0].astype(np.int64) << 7)
    assert np.array_equal(E16, np.where(x8[1] == E_ZERO_, E_ZERO_, x8[1].astype(np.int64) - 7))
    # R16 inputs with full 15-bit mantissas and exponents spread around the INT8 addend's
    xm = R.uniform_int(92, (Rn, C), -32767, 32767)
    xm[:, :blk] //= 300                                      # a block with small mantissas (not normalized)
    xE = R.uniform_int(93, (Rn, C // blk), -20, 20)
    zx = R.uniform01(94, (Rn, C // blk)) < 0.05
    xm.reshape(Rn, C // blk, blk)[zx] = 0
    xE[zx] = E_ZERO_
    ym, yE = R.bloco(95, Rn, C, blk, espalha=30, e0=-5, zera=0.1)
    X16 = (t(xm.astype(np.int16)), t(xE.astype(np.int8)))
    Y = (t(ym), t(yE))
    z = ops.soma16(X16, Y)
    zm, zE = host(z[0]).astype(np.int64).reshape(-1), host(z[1]).astype(np.int64).reshape(-1)
    p8 = ops.para8(X16)
    pm, pE = host(p8[0]).astype(np.int64).reshape(-1), host(p8[1]).astype(np.int64).reshape(-1)
    for r in range(Rn):
        V, S, V8, S8 = [], [], [], []
        for b in range(C // blk):
            ex, ey = int(xE[r, b]), int(yE[r, b])
            for k in range(b * blk, (b + 1) * blk):
                xv = int(xm[r, k]) if ex != E_ZERO_ else 0
                yv = int(ym[r, k]) if ey != E_ZERO_ else 0
                s0 = min(ex, ey)
                V.append((xv << (ex - s0)) + (yv << (ey - s0)))
                S.append(s0)
                V8.append(xv)
                S8.append(ex)
        mq, Eq = _quant_exata(V, S, 15, 32767, blk)
        assert list(zm[r * C:(r + 1) * C]) == mq and list(zE[r * (C // blk):(r + 1) * (C // blk)]) == Eq, f"soma16 row {r}"
        mq, Eq = _quant_exata(V8, S8, 7, 127, blk)
        assert list(pm[r * C:(r + 1) * C]) == mq and list(pE[r * (C // blk):(r + 1) * (C // blk)]) == Eq, f"para8 row {r}"


@pytest.mark.parametrize("desloc", [0, 32, 60])
@pytest.mark.parametrize("limite", [False, True])
def test_atencao_hd64_reduz_ao_spec_hd4(limite, desloc):
    """The head-width-64 attention (the declared extension run at configs 4 and 5) on inputs where each head
    carries one head-width-4 head of the spec's shape in its dimensions desloc .. desloc + 3 (tests/reducoes.py,
    family 1) gives that head's outputs: P, o and, in the backward (both variants), gq, gk, gv. The head-width-4
    side is the oracle code the reference's goldens pin (ops.py:186-258). This pins the extension's alignment
    over a head's blocks (desloc 32 and 60: the data in the head's second block, its first block all-zero), its
    score shift -(log2 hd)/2, its ALiBi schedule 8 - 8h/H and its backward at T <= 128."""
    import reducoes as RD
    Bt, T = 2, 128
    ops = OpsOraculo(32, limite=limite)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    (q4, g4), (q64, g64) = RD.problemas(5150 + desloc, Bt, T, desloc)
    Q4, G4, Q64, G64 = [tuple(t(v) for v in x) for x in (q4, g4, q64, g64)]
    f4, f64 = ops.atencao(Q4, Bt, T, RD.H4), ops.atencao(Q64, Bt, T, RD.H64)
    RD.confere_frente([[host(x) for x in f4[0]], host(f4[1])], [[host(x) for x in f64[0]], host(f64[1])], Bt, desloc)
    b4 = ops.atencao_back(G4, Q4, f4[1], Bt, T, RD.H4)
    b64 = ops.atencao_back(G64, Q64, f64[1], Bt, T, RD.H64)
    RD.confere_tras([host(x) for x in b4], [host(x) for x in b64], desloc)


@pytest.mark.parametrize("limite", [False, True])
def test_atencao_hd64_tras_v_zero(limite):
    """Head width 64 at config 4's shape (8 heads x 64, T = 256, BLK = 32) with v = 0 and q, k, dO random in all
    64 dimensions of both blocks (tests/reducoes.py, family 2). Then gP = dO v^T = 0, so s_lin = dS = 0 and
    (ops.py:221-258, both variants):
      * gq = gk = 0 exactly, at exponents eds + ek and eds + eq with eds = ego + ev - 9 (both shrink counts 0);
      * gv_j = sum_i P_ij a_i over every dimension, a = dO aligned to the head's largest block exponent over
        both blocks and T tokens (exact half-even rounding), at exponent ego - 8;
      * and, independently of any rounding rule, gv 2^(ego - 8) is within sum_i P_ij 2^(ego - 1) / 256 of the
        exact sum_i (P_ij / 256) dO_i (each aligned value is within half its ulp 2^ego of dO_i)."""
    import reducoes as RD
    Bt, T, H, D, blk, GA = 2, 256, 8, 512, 32, 4
    (qm, qE), (gm, gE) = RD.problema_v_zero(7310, Bt, T)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    ops = OpsOraculo(blk, limite=limite)
    _, P = ops.atencao((t(qm), t(qE)), Bt, T, H)
    acc, e = (host(x).astype(np.int64) for x in ops.atencao_back((t(gm), t(gE)), (t(qm), t(qE)), P, Bt, T, H))
    P = host(P)
    assert np.count_nonzero(P) > Bt * H * T                     # P is not trivial
    assert not np.any(acc[:, :2 * D]), "gq, gk must be 0"
    gv, expo = RD.gv_v_zero((gm, gE), P, Bt, T)
    assert np.array_equal(acc[:, 2 * D:], gv), "gv"
    assert np.count_nonzero(gv[:, 64 * np.arange(H)[:, None] + np.arange(4, 64)[None, :]]) > 0.9 * Bt * T * H * 60
    Pb = P.astype(np.int64).reshape(Bt, H, T, T)
    qE64, gE64 = qE.astype(np.int64), gE.astype(np.int64)
    for b in range(Bt):
        rows = slice(b * T, (b + 1) * T)
        for h in range(H):
            cols = slice(64 * h, 64 * (h + 1))
            emx = lambda E, part: int(E[rows, part * (D // blk) + 2 * h:part * (D // blk) + 2 * h + 2].max())
            ego, eq, ek, ev = emx(gE64, 0) - GA, emx(qE64, 0) - GA, emx(qE64, 1) - GA, -127 - GA
            eds = ego + ev - 9
            assert ev == emx(qE64, 2) - GA
            assert np.all(e[rows, cols] == eds + ek) and np.all(e[rows, D:][:, cols] == eds + eq), (b, h, "gq/gk e")
            assert np.all(e[rows, 2 * D:][:, cols] == expo[b, h]) and expo[b, h] == ego - 8, (b, h, "gv e")
            # float bound (exact in float64: 256 terms of 2^15 x 2^E over a 12-step exponent range)
            x = gm[rows, cols].astype(np.float64) * np.exp2(np.repeat(gE64[rows, 2 * h:2 * h + 2], blk, 1))
            exato = Pb[b, h].astype(np.float64) @ x / 256.0
            folga = Pb[b, h].sum(1).astype(np.float64)[:, None] * 2.0 ** (ego - 1) / 256.0
            assert np.all(np.abs(gv[rows, cols] * 2.0 ** (ego - 8) - exato) <= folga), (b, h, "gv bound")


@pytest.mark.parametrize("limite", [False, True])
def test_atencao_hd64_permutacao(limite):
    """Head width 64 at config 4's shape with one exponent per (token, head) on both blocks of q, k, v and dO
    (tests/reducoes.py, family 3): permuting every head's q and k dimensions jointly by pi[h] and its v and dO
    dimensions by sigma[h] (across both blocks) leaves P unchanged and permutes o and gv by sigma and gq, gk by
    pi, values and exponents, bit for bit, in both backward variants. An oracle that drops, repeats or
    misindexes any dimension of 4 .. 63, or treats the second block differently, fails it."""
    import reducoes as RD
    Bt, T, H, D, blk = 2, 256, 8, 512, 32
    (qkv, go), (qkv_p, go_p), pi, sigma = RD.problema_permutado(7311, Bt, T)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    ops = OpsOraculo(blk, limite=limite)
    saidas = []
    for q, g in ((qkv, go), (qkv_p, go_p)):
        (oacc, oe), P = ops.atencao(tuple(t(v) for v in q), Bt, T, H)
        ga, ge = ops.atencao_back(tuple(t(v) for v in g), tuple(t(v) for v in q), P, Bt, T, H)
        saidas.append([host(x) for x in (oacc, oe, P, ga, ge)])
    (oa, oe, P, ga, ge), (oa_p, oe_p, P_p, ga_p, ge_p) = saidas
    assert np.array_equal(P, P_p), "P"
    assert np.array_equal(oa_p, RD.permuta_colunas(oa, sigma, D, 0)), "o"
    assert np.array_equal(oe_p, RD.permuta_colunas(oe, sigma, D, 0)), "o exponents"
    for x, x_p, nome in ((ga, ga_p, "acc"), (ge, ge_p, "e")):
        y = RD.permuta_colunas(RD.permuta_colunas(RD.permuta_colunas(x, pi, D, 0), pi, D, 1), sigma, D, 2)
        assert np.array_equal(x_p, y), f"backward {nome}"
    assert np.count_nonzero(ga[:, :2 * D]) > 0.5 * ga[:, :2 * D].size    # dS is not trivial


def test_atencao_hd64_q_zero_so_alibi():
    """With q = 0 every score is the ALiBi term alone, u_ij = -((i - j) << (8 - 8h/H)): P has the closed form
    min((e_ij (2^28 // sum_j e_ij) + 2^19) >> 20, 255), e_ij = exp_int((i - j) << incl) >> 3 (exp_int pinned by
    primitives.json), for every head of the head-width-64 problem (H = 8: slopes 2^0 .. 2^-7), T = 256."""
    Bt, T, H, D, blk = 1, 256, 8, 512, 32
    m = R.uniform_int(97, (Bt * T, 3 * D), -127, 127).astype(np.int8)
    m[:, :D] = 0
    E = R.uniform_int(98, (Bt * T, 3 * D // blk), -9, -3).astype(np.int8)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    (_, _), P = OpsOraculo(blk).atencao((t(m), t(E)), Bt, T, H)
    P = host(P).reshape(H, T, T)                               # [h][j][i]
    ex = OpsOraculo.prim("exp_int", np.arange(0, 256 << 8))
    for h in range(H):
        incl = 8 - (8 * h) // H
        for i in (0, 1, 37, 128, 255):
            e = [int(ex[min((i - j) << incl, len(ex) - 1)]) >> 3 for j in range(i + 1)]
            inv = (1 << 28) // sum(e)
            esperado = [min((v * inv + (1 << 19)) >> 20, 255) for v in e] + [0] * (T - i - 1)
            assert list(P[h, :, i]) == esperado, (h, i)


def test_atencao_hd64_k_um_quente():
    """Head width 64 with one-hot keys (token j's k is c_j in dimension j % 64 and 0 elsewhere) and every q, k, v block
    of a head at one exponent, so alignment is exact (a = m << 4): then q.k_j = 256 q_i[j % 64] c_j, and the score
    is u_ij = rnd(256 q_i[j % 64] c_j, -(eq + ek - log2(64)/2 + 8)) - ((i - j) << (8 - 8h/H)) with eq, ek the
    exponents minus GA = 4 (round half even, here as exact Fraction rounding); P follows from u by the spec's softmax
    (exp_int pinned by primitives.json), and o = sum_j P_ij (v_j << 4) at exponent ev - 8. At e_q + e_k = -7 the
    shift is 10 bits, so half-even rounding and the -(log2 hd)/2 term both decide bits of u."""
    from fractions import Fraction
    Bt, T, H, D, blk, GA = 1, 128, 8, 512, 32, 4
    eqb, ekb, evb = -3, -4, -6
    q = R.uniform_int(111, (T, D), -127, 127)
    c = R.uniform_int(112, (T,), 1, 127) * np.where(R.uniform01(113, (T,)) < 0.5, -1, 1)
    v = R.uniform_int(114, (T, D), -127, 127)
    m = np.zeros((Bt * T, 3 * D), np.int64)
    m[:, :D] = q
    m[:, 2 * D:] = v
    for h in range(H):
        for j in range(T):
            m[j, D + 64 * h + j % 64] = c[j]
    E = np.empty((Bt * T, 3 * D // blk), np.int64)
    E[:, :D // blk], E[:, D // blk:2 * D // blk], E[:, 2 * D // blk:] = eqb, ekb, evb
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    (oacc, oe), P = OpsOraculo(blk).atencao((t(m.astype(np.int8)), t(E.astype(np.int8))), Bt, T, H)
    P, oacc, oe = host(P).reshape(H, T, T), host(oacc).astype(np.int64), host(oe).astype(np.int64)
    ex = OpsOraculo.prim("exp_int", np.arange(0, 1 << 17))
    su = -((eqb - GA) + (ekb - GA) - 3 + 8)
    assert su == 10
    for h in range(H):
        incl = 8 - (8 * h) // H
        for i in (0, 5, 63, 64, 100, 127):
            u = [round(Fraction(256 * int(q[i, 64 * h + j % 64]) * int(c[j]), 1 << su)) - ((i - j) << incl)
                 for j in range(i + 1)]
            mx = max(u)
            e = [int(ex[mx - x]) >> 3 for x in u]
            inv = (1 << 28) // sum(e)
            p = [min((x * inv + (1 << 19)) >> 20, 255) for x in e]
            assert list(P[h, :, i]) == p + [0] * (T - i - 1), (h, i)
            for d in (0, 17, 63):
                o = sum(p[j] * (int(v[j, 64 * h + d]) << GA) for j in range(i + 1))
                assert oacc[i, 64 * h + d] == o and oe[i, 64 * h + d] == (evb - GA) - 8, (h, i, d)


def test_largura_de_ds_por_t():
    """The attention backward shrinks dS to 12 - max(0, ceil(log2 T) - 7) bits past T = 128 (jatai_oracle.cpp
    att_dsbits, the kernels' ds_bits). The spec fixes 12 bits for T <= 128 (ops.py:245-247), where its int32 proof
    bounds |gq|, |gk| = |sum_j dS_ij a_j| by T (2^12 - 1) 2032 < 2^30 (a: aligned values, |a| <= 127 << GA = 2032;
    RELATORIO_TECNICO.md:897-927). The oracle's rule keeps that bound at every T the kernels accept (T % 32 up to
    256, T % 64 up to 512), is the spec's 12 bits up to 128, and is the widest width that does so at T = 128, 256
    and 512: one bit more would break the bound there."""
    from oracle import ops_oracle as OO
    largura = OO.lib().or_att_dsbits
    lim, amax = 1 << 30, 127 << OO.GA
    for T in range(32, 513, 32):
        dsb = largura(T)
        assert 0 < dsb <= 12, T
        assert T * ((1 << dsb) - 1) * amax < lim, (T, dsb)
        if T <= 128:
            assert dsb == 12, T
        if T in (128, 256, 512):
            assert T * ((1 << (dsb + 1)) - 1) * amax >= lim, (T, dsb)
        if T > 32:
            assert dsb <= largura(T - 32), T                  # never wider for a longer sequence


@pytest.mark.parametrize("blk", [32, 128])
def test_de_f32_exato(blk):
    """The fp32 data path (BASELINE configs 2 and 3: fp32 N(0, 1) activations quantized to blocks): frexp splits
    every float32 exactly (v 2^e == x, |v| < 2^24), and the oracle's block tensor is the spec's quantization rule
    applied to those exact values (_quant_exata, exact integer rounding), including zeros, subnormals and values
    far apart within a block."""
    ops = OpsOraculo(blk)
    Rn, C = 16, 4 * blk
    x = R.normal32(401, (Rn, C))
    x[0, :blk] = 0.0                                           # a zero block
    x[1, :5] = np.array([1e-40, -3e-39, 0.0, 2.5e-45, 7.0], np.float32)   # subnormals beside a normal value
    x[2, :blk] *= np.float32(2.0 ** 60)                        # a block of large values
    x[3, ::7] = np.float32(1e-30)                              # tiny values among normal ones
    m, e = np.frexp(x)
    v = (m.astype(np.float64) * 2.0 ** 24).astype(np.int64)
    assert np.array_equal(np.ldexp(v.astype(np.float64), (e - 24).astype(np.int64)), x.astype(np.float64))
    assert np.all(np.abs(v) < 1 << 24)
    qm, qE = (host(t).astype(np.int64) for t in ops.de_f32(torch.from_numpy(x)))
    for r in range(Rn):
        ms, Es = _quant_exata([int(a) for a in v[r]], [int(a) - 24 for a in e[r]], 7, 127, blk)
        assert list(qm[r]) == ms and list(qE[r]) == Es, f"row {r}"
    with pytest.raises(ValueError):
        ops.de_f32(torch.from_numpy(np.full((1, blk), np.inf, np.float32)))
