"""The op-level parity cases, written once and run against any backend with the reference operator surface.

The list mirrors the reference's 40 distinct cases in `jatai_cuda/teste_ops.py:57-98` (there run twice for the
two GEMM tiles, 53 runs in all), at the reference's model sizes `teste_ops.py:55` (Bt=8, T=128, H=64, D=256,
FF=1024, V=256). Inputs come from `recipe.py` (portable SplitMix64) instead of torch's RNG, so the same case
gives the same bytes in the fixture writer and in every test.

A backend adapter provides: `ops` (an object with the reference's methods), `dev(np_array)` -> backend tensor,
`host(tensor)` -> numpy, and `limite(flag)` to toggle the attention-backward bound variant.
"""
import numpy as np

import recipe as R

Bt, T, H, D, FF, V = 8, 128, 64, 256, 1024, 256
M = Bt * T


class Gen:
    """Lazily numbered inputs: the k-th input of a case uses substream(case_seed, k)."""

    def __init__(self, seed, blk, dev):
        self.seed, self.k, self.blk, self.dev = seed, 0, blk, dev

    def _next(self):
        self.k += 1
        return R.substream(self.seed, self.k)

    def bloco(self, Rr, C, **kw):
        m, E = R.bloco(self._next(), Rr, C, self.blk, **kw)
        return self.dev(m), self.dev(E)

    def cru(self, Rr, C, **kw):
        acc, e = R.cru(self._next(), Rr, C, **kw)
        return self.dev(acc), self.dev(e)

    def tok(self, n, Vv):
        return self.dev(R.tokens(self._next(), n, Vv))

    def zeros_cru(self, Rr, C):
        return self.dev(np.zeros((Rr, C), np.int32)), self.dev(np.zeros((Rr, C), np.int16))

    def zeros_bloco(self, Rr, C):
        return self.dev(np.zeros((Rr, C), np.int8)), self.dev(np.full((Rr, C // self.blk), R.E_ZERO, np.int8))


def casos():
    """(name, fn(ops, gen, be)) in the reference order. `be.limite` toggles ATENCAO_LIMITE."""
    c = []
    a = c.append
    # ---- GEMM family (teste_ops.py:58-70)
    a(("gemm Q x Wqkv", lambda o, g, be: o.gemm(g.bloco(M, D), g.bloco(3 * D, D))))
    a(("gemm tile 128 (M=2048, N=1024)", lambda o, g, be: o.gemm(g.bloco(2 * M, D, espalha=6), g.bloco(FF, D))))
    a(("gemm tile 128 cru", lambda o, g, be: o.gemm(g.bloco(2 * M, D), g.bloco(FF, D), cru=True)))
    a(("gemm com blocos zerados", lambda o, g, be: o.gemm(g.bloco(M, D, zera=0.3), g.bloco(D, D, zera=0.3))))
    a(("gemm K=1024 expoentes espalhados", lambda o, g, be: o.gemm(g.bloco(M, FF, espalha=12), g.bloco(D, FF, espalha=12))))
    a(("gemm cru (grad de peso, K=tokens)", lambda o, g, be: o.gemm(g.bloco(D, M), g.bloco(FF, M), cru=True)))
    a(("gemm cru split-K em 8 partes", lambda o, g, be: o.gemm(g.bloco(D, M, espalha=8), g.bloco(D, M, espalha=8), cru=True)))
    a(("gemm cru split-K com blocos zerados", lambda o, g, be: o.gemm(g.bloco(D, M, zera=0.4), g.bloco(3 * D, M, zera=0.4), cru=True)))
    a(("gemm + soma residual", lambda o, g, be: o.gemm_soma(g.bloco(M, D), g.bloco(D, D), g.bloco(M, D, espalha=10, zera=0.1))))
    a(("gemm + soma, residuo muito maior/menor",
       lambda o, g, be: o.gemm_soma(g.bloco(M, FF), g.bloco(D, FF), g.bloco(M, D, e0=8, espalha=20, zera=0.2))))
    a(("gemm + relu2", lambda o, g, be: o.gemm_relu2(g.bloco(M, D, zera=0.1), g.bloco(FF, D))))
    a(("gemm + relu2 com underflow", lambda o, g, be: o.gemm_relu2(g.bloco(M, D, e0=-40), g.bloco(FF, D, e0=-40))))
    a(("gemm + relu2_back", lambda o, g, be: o.gemm_relu2_back(g.bloco(M, D), g.bloco(FF, D), g.bloco(M, FF, zera=0.1))))
    # ---- element-wise, reductions, attention, optimizer (teste_ops.py:71-97)
    a(("transpoe", lambda o, g, be: o.transpoe(g.bloco(M, 3 * D, espalha=8, zera=0.1))))
    a(("quant", lambda o, g, be: o.quant(g.cru(M, D))))
    a(("quant com zeros", lambda o, g, be: o.quant(g.zeros_cru(M, D))))
    a(("soma", lambda o, g, be: o.soma(g.bloco(M, D, espalha=10, zera=0.1), g.bloco(M, D, espalha=10, zera=0.1))))
    a(("relu2", lambda o, g, be: o.relu2(g.bloco(M, FF, zera=0.1))))
    a(("relu2_back", lambda o, g, be: o.relu2_back(g.bloco(M, FF), g.bloco(M, FF))))
    a(("um_quente", lambda o, g, be: o.um_quente(g.tok(M, V), V)))
    a(("embed", lambda o, g, be: o.embed(g.bloco(V, D), g.tok(M, V))))
    a(("rms", lambda o, g, be: o.rms(g.bloco(M, D, espalha=6, zera=0.2))))
    a(("rms com mantissas pequenas", lambda o, g, be: o.rms(g.bloco(M, D, mmax=3))))
    a(("rms_back", lambda o, g, be: (lambda Y: o.rms_back(g.bloco(M, D, espalha=6), Y[0], Y[1]))(o.rms(g.bloco(M, D)))))
    a(("atencao", lambda o, g, be: o.atencao(g.bloco(M, 3 * D, espalha=3), Bt, T, H)))
    a(("atencao softmax concentrado", lambda o, g, be: o.atencao(g.bloco(M, 3 * D, e0=-3), Bt, T, H)))
    a(("atencao shift do score a esquerda <= 6", lambda o, g, be: o.atencao(g.bloco(M, 3 * D, e0=0, espalha=1), Bt, T, H)))
    a(("atencao shift do score a esquerda > 6",
       lambda o, g, be: o.atencao(g.bloco(M, 3 * D, e0=4, espalha=1, mmax=3), Bt, T, H)))
    a(("atencao expoentes muito espalhados", lambda o, g, be: o.atencao(g.bloco(M, 3 * D, espalha=12, zera=0.1), Bt, T, H)))
    a(("atencao_back expoentes muito espalhados", lambda o, g, be: _att_back(o, g, be, dict(e0=-20, espalha=12, zera=0.1),
                                                                           dict(espalha=12, zera=0.1), False)))
    a(("atencao_back variante limite", lambda o, g, be: _att_back(o, g, be, dict(e0=-20), dict(), True)))
    a(("atencao_back variante limite, expoentes espalhados",
       lambda o, g, be: _att_back(o, g, be, dict(e0=-20, espalha=12, zera=0.1), dict(espalha=12, zera=0.1), True)))
    a(("atencao_back", lambda o, g, be: _att_back(o, g, be, dict(e0=-20), dict(), False)))
    a(("softmax_ce", lambda o, g, be: o.softmax_ce(g.cru(M, V, bits=22, e0=-20), g.tok(M, V))))
    a(("momento", lambda o, g, be: o.momento(g.cru(D, D, bits=28, e0=-50), g.bloco(D, D, e0=-40))))
    a(("momento caindo abaixo de 2^-126", lambda o, g, be: o.momento(g.zeros_cru(D, D), g.bloco(D, D, e0=-122, espalha=3))))
    a(("momento a partir de zero", lambda o, g, be: o.momento(g.cru(D, D, bits=20), g.zeros_bloco(D, D))))
    a(("peso com error feedback", lambda o, g, be: o.peso(g.bloco(D, D, e0=-9), g.bloco(D, D, e0=-15),
                                                            g.bloco(D, D, e0=-20, zera=0.3), 4, True)))
    a(("peso sem error feedback", lambda o, g, be: o.peso(g.bloco(D, D, e0=-9), g.bloco(D, D, e0=-15), g.bloco(D, D), 4, False)))
    a(("peso com passo maior que o peso", lambda o, g, be: o.peso(g.bloco(D, D, e0=-12), g.bloco(D, D, e0=-2),
                                                                    g.bloco(D, D, e0=-20), 1, True)))
    return c


def casos_dominio():
    """The rest of the reference's shape domain, beyond the model shape of casos(): rms / rms_back at widths that
    are multiples of 128 but not powers of two (ops.py:453, D <= 1024), softmax_ce at V = 384 and 640
    (ops.py:496, V % 128 == 0), and head-width-4 attention at H = 32 and at T = 32 and 96 (ops.py:475:
    T % 32 == 0, T <= 128, H * 4 == D, H <= 64). Same generators as casos()."""
    c = []
    a = c.append
    Mr = 256
    for Dd in (384, 640, 768, 896):
        a((f"rms D={Dd}", lambda o, g, be, Dd=Dd: o.rms(g.bloco(Mr, Dd, espalha=6, zera=0.1))))
    for Dd in (384, 896):
        a((f"rms_back D={Dd}", lambda o, g, be, Dd=Dd: (lambda Y: o.rms_back(g.bloco(Mr, Dd, espalha=6), Y[0], Y[1]))(
            o.rms(g.bloco(Mr, Dd)))))
    for Vv in (384, 640):
        a((f"softmax_ce V={Vv}", lambda o, g, be, Vv=Vv: o.softmax_ce(g.cru(Mr, Vv, bits=22, e0=-20), g.tok(Mr, Vv))))
    for (bt, t, h) in ((4, 96, 32), (8, 32, 64), (2, 128, 32)):
        dd = 4 * h
        a((f"atencao Bt={bt} T={t} H={h}", lambda o, g, be, bt=bt, t=t, h=h, dd=dd:
           o.atencao(g.bloco(bt * t, 3 * dd, espalha=3), bt, t, h)))
        for lim in (False, True):
            a((f"atencao_back Bt={bt} T={t} H={h}" + (" limite" if lim else ""),
               lambda o, g, be, bt=bt, t=t, h=h, dd=dd, lim=lim: _att_back_forma(o, g, be, bt, t, h, dd, lim)))
    return c


def _att_back_forma(o, g, be, bt, t, h, dd, limite):
    q = g.bloco(bt * t, 3 * dd, espalha=6, zera=0.05)
    go = g.bloco(bt * t, dd, e0=-20, espalha=6)
    P = o.atencao(q, bt, t, h)[1]
    old = be.limite(limite)
    try:
        return o.atencao_back(go, q, P, bt, t, h)
    finally:
        be.limite(old)


def _att_back(o, g, be, go_kw, q_kw, limite):
    """atencao_back on P from the same backend's forward (teste_ops.py:87-90: q drawn first, then dO)."""
    q = g.bloco(M, 3 * D, **q_kw)
    go = g.bloco(M, D, **go_kw)
    P = o.atencao(q, Bt, T, H)[1]
    old = be.limite(limite)
    try:
        return o.atencao_back(go, q, P, Bt, T, H)
    finally:
        be.limite(old)


def plano(x):
    """Flatten nested tuples of tensors, in order."""
    if isinstance(x, (tuple, list)):
        return [t for y in x for t in plano(y)]
    return [x]


class Gravador:
    """Wraps an ops object: every call's outputs are recorded as (op, [sha256 per output]) in call order.
    In-place ops (momento, peso) are hashed after the call, like the reference checker compares them
    (ops.py:557-562)."""

    def __init__(self, ops, host):
        self._ops, self._host, self.log = ops, host, []

    def __getattr__(self, op):
        f = getattr(self._ops, op)
        if not callable(f):
            return f

        def g(*a, **kw):
            out = f(*a, **kw)
            self.log.append((op, [R.sha(self._host(t)) for t in plano(out)]))
            return out
        return g
