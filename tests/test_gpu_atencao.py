"""Attention at head width 64 (the BASELINE configs' 8 heads x 64 of D = 512, T = 256): the HIP kernels against
the CPU oracle's generalized restatement (jatai_oracle.cpp, which reduces to the spec at head width 4, pinned by
the golden fixtures). Bit-exact: P, the raw output (acc, e), and the backward's raw (acc, e) in both variants.
The generalization has no reference counterpart; test_atencao_hd64_reduz_ao_spec_hd4 pins it to the spec's
head-width-4 arithmetic on inputs where the two problems coincide (T <= 128)."""
import numpy as np
import pytest
import torch

import recipe as R
from backends import CPU, GPU, host, primeira_diferenca

pytestmark = pytest.mark.gpu


def _cmp(a, b, nome):
    a, b = (x if isinstance(x, np.ndarray) else host(x) for x in (a, b))
    d = primeira_diferenca(a, b)
    assert d is None, f"{nome}: (flat index, gpu, oracle, count) = {d}"


@pytest.fixture(params=["ws", "abi", "dot2"])
def via_ws(request):
    """ws: OpsHip's default path (jt_atencao_ws, workspace kernels at head width 64); abi: the reference ABI's
    jt_atencao (matrix-core kernels that stage their own operands); dot2: the same entry points with
    jt_atencao_mfma(0), the v_dot2 kernel family."""
    from jatai_amd import ops as O
    lib = O.carrega_lib()
    old = O.ATENCAO_WS
    O.ATENCAO_WS = request.param == "ws"
    if request.param == "dot2":
        lib.jt_atencao_mfma(0)
    try:
        yield request.param
    finally:
        O.ATENCAO_WS = old
        lib.jt_atencao_mfma(1)


# exponents e0 +- espalha stay in the range where the int32 sentinels stay silent (e0 + espalha <= 2, as the
# reference's own spread cases, teste_ops.py:86-87); GPU() reads the device error record after every op
@pytest.mark.parametrize("blk,Bt,T,H,D,esp,e0,limite", [
    (32, 2, 256, 8, 512, 3, -7, False),
    (32, 2, 256, 8, 512, 10, -9, True),
    (128, 2, 128, 8, 512, 6, -7, False),
    (32, 1, 256, 4, 256, 12, -10, True),
    (32, 2, 128, 16, 512, 2, -7, False),
    (32, 1, 512, 4, 256, 3, -7, False),
    (32, 1, 192, 4, 256, 3, -7, False),
], ids=["cfg4", "cfg4-limite-espalhado", "blk128-T128", "H4-espalhado-limite", "hd32", "T512", "T192"])
def test_atencao_hd_vs_oraculo(blk, Bt, T, H, D, esp, e0, limite, via_ws):
    M = Bt * T
    seed = R.substream(555, f"{blk} {Bt} {T} {H} {D} {esp} {limite}")
    qn = R.bloco(R.substream(seed, "qkv"), M, 3 * D, blk, espalha=esp, e0=e0, zera=0.05)
    gn = R.bloco(R.substream(seed, "go"), M, D, blk, espalha=esp, e0=-20, zera=0.05)
    res = []
    for be in (GPU(blk, vigiar=True), CPU(blk)):
        qkv = tuple(be.dev(v) for v in qn)
        go = tuple(be.dev(v) for v in gn)
        (oacc, oe), P = be.ops.atencao(qkv, Bt, T, H)
        old = be.limite(limite)
        try:
            gacc, ge = be.ops.atencao_back(go, qkv, P, Bt, T, H)
        finally:
            be.limite(old)
        res.append((oacc, oe, P, gacc, ge))
    for nome, a, b in zip(("oacc", "oe", "P", "gacc", "ge"), *res):
        _cmp(a, b, nome)


@pytest.mark.parametrize("T,H,limite", [(256, 8, False), (256, 8, True), (512, 4, False)])
def test_atencao_q_igual_a_quant(T, H, limite):
    """atencao_q / atencao_back_q (outputs quantized inside the attention kernels) equal quant of the raw outputs."""
    blk, Bt, D = 32, 2, 64 * H
    gpu = GPU(blk, vigiar=True)
    seed = R.substream(556, f"q {T} {H} {limite}")
    qkv = tuple(gpu.dev(v) for v in R.bloco(R.substream(seed, "qkv"), Bt * T, 3 * D, blk, espalha=4, e0=-7, zera=0.05))
    go = tuple(gpu.dev(v) for v in R.bloco(R.substream(seed, "go"), Bt * T, D, blk, espalha=4, e0=-20, zera=0.05))
    o = gpu.ops
    old = gpu.limite(limite)
    try:
        om, P = o.atencao_q(qkv, Bt, T, H)
        oc, P2 = o.atencao(qkv, Bt, T, H)
        ref = o.quant(oc)
        gq = o.atencao_back_q(go, qkv, P, Bt, T, H)
        gref = o.quant(o.atencao_back(go, qkv, P, Bt, T, H))
    finally:
        gpu.limite(old)
    for nome, a, b in (("om", om[0], ref[0]), ("omE", om[1], ref[1]), ("P", P, P2), ("gq", gq[0], gref[0]), ("gqE", gq[1], gref[1])):
        _cmp(a, b, nome)


@pytest.mark.parametrize("T,H,limite", [(256, 8, False), (256, 8, True), (512, 4, False), (64, 2, False), (128, 16, False)])
def test_atencao_qs_igual_a_q(T, H, limite):
    """atencao_qs / atencao_back_qs (q, k, v converted for the backward by the forward's pass and read back from the
    saved buffer; the bound variant converts them again) equal atencao_q / atencao_back_q, also on a second backward
    from the same buffer."""
    blk, Bt, D = 32, 2, 64 * H
    gpu = GPU(blk, vigiar=True)
    seed = R.substream(557, f"qs {T} {H} {limite}")
    qkv = tuple(gpu.dev(v) for v in R.bloco(R.substream(seed, "qkv"), Bt * T, 3 * D, blk, espalha=4, e0=-7, zera=0.05))
    go = tuple(gpu.dev(v) for v in R.bloco(R.substream(seed, "go"), Bt * T, D, blk, espalha=4, e0=-20, zera=0.05))
    go2 = tuple(gpu.dev(v) for v in R.bloco(R.substream(seed, "go2"), Bt * T, D, blk, espalha=4, e0=-18, zera=0.05))
    o = gpu.ops
    old = gpu.limite(limite)
    try:
        om, P, sv = o.atencao_qs(qkv, Bt, T, H)
        assert sv is not None
        om_r, P_r = o.atencao_q(qkv, Bt, T, H)
        gq = o.atencao_back_qs(go, qkv, P, sv, Bt, T, H)
        gq2 = o.atencao_back_qs(go2, qkv, P, sv, Bt, T, H)
        gq_r = o.atencao_back_q(go, qkv, P, Bt, T, H)
        gq2_r = o.atencao_back_q(go2, qkv, P, Bt, T, H)
    finally:
        gpu.limite(old)
    for nome, a, b in (("om", om[0], om_r[0]), ("omE", om[1], om_r[1]), ("P", P, P_r), ("gq", gq[0], gq_r[0]), ("gqE", gq[1], gq_r[1]),
                       ("gq2", gq2[0], gq2_r[0]), ("gq2E", gq2[1], gq2_r[1])):
        _cmp(a, b, nome)


def _frente_tras(be, qn, gn, Bt, T, H, limite):
    """(oacc, oe, P, gacc, ge) of one forward and backward on a backend, as host arrays."""
    qkv = tuple(be.dev(v) for v in qn)
    go = tuple(be.dev(v) for v in gn)
    old = be.limite(limite)
    try:
        (oacc, oe), P = be.ops.atencao(qkv, Bt, T, H)
        gacc, ge = be.ops.atencao_back(go, qkv, P, Bt, T, H)
    finally:
        be.limite(old)
    return [host(x) for x in (oacc, oe, P, gacc, ge)]


@pytest.mark.parametrize("limite", [False, True])
def test_atencao_hd64_tras_v_zero(limite, via_ws):
    """Config 4's attention shape with v = 0 and q, k, dO random in every dimension of both blocks
    (tests/reducoes.py, family 2): each kernel family gives gq = gk = 0 and gv = sum_i P_ij a_i over all 64
    dimensions (the closed form), and every output equals the oracle's."""
    import reducoes as RD
    Bt, T, H = 2, 256, 8
    qn, gn = RD.problema_v_zero(7310, Bt, T)
    g = _frente_tras(GPU(32, vigiar=True), qn, gn, Bt, T, H, limite)
    c = _frente_tras(CPU(32), qn, gn, Bt, T, H, limite)
    acc = g[3].astype(np.int64)
    assert not np.any(acc[:, :2 * RD.D64]), "gq, gk must be 0"
    gv, _ = RD.gv_v_zero(gn, g[2], Bt, T)
    assert np.array_equal(acc[:, 2 * RD.D64:], gv), "gv closed form"
    for nome, a, b in zip(("oacc", "oe", "P", "gacc", "ge"), g, c):
        _cmp(a, b, nome)


@pytest.mark.parametrize("limite", [False, True])
def test_atencao_hd64_permutacao(limite, via_ws):
    """Config 4's attention shape with one exponent per (token, head) on both blocks (tests/reducoes.py, family 3):
    permuting each head's q, k dimensions by pi and v, dO dimensions by sigma permutes each kernel family's o, gv
    by sigma and gq, gk by pi and leaves P unchanged, bit for bit; the unpermuted outputs equal the oracle's."""
    import reducoes as RD
    Bt, T, H, D = 2, 256, 8, 512
    (qn, gn), (qp, gp), pi, sigma = RD.problema_permutado(7311, Bt, T)
    gpu = GPU(32, vigiar=True)
    a = _frente_tras(gpu, qn, gn, Bt, T, H, limite)
    b = _frente_tras(gpu, qp, gp, Bt, T, H, limite)
    c = _frente_tras(CPU(32), qn, gn, Bt, T, H, limite)
    for nome, x, y in zip(("oacc", "oe", "P", "gacc", "ge"), a, c):
        _cmp(x, y, nome)
    _cmp(b[2], a[2], "P permuted")
    _cmp(b[0], RD.permuta_colunas(a[0], sigma, D, 0), "o permuted")
    _cmp(b[1], RD.permuta_colunas(a[1], sigma, D, 0), "o exponents permuted")
    for i, nome in ((3, "acc"), (4, "e")):
        y = RD.permuta_colunas(RD.permuta_colunas(RD.permuta_colunas(a[i], pi, D, 0), pi, D, 1), sigma, D, 2)
        _cmp(b[i], y, f"backward {nome} permuted")
    assert np.count_nonzero(a[3][:, :2 * D]) > 0.5 * a[3][:, :2 * D].size


@pytest.mark.parametrize("desloc", [0, 32, 60])
@pytest.mark.parametrize("limite", [False, True])
def test_atencao_hd64_reduz_ao_spec_hd4(limite, desloc, via_ws):
    """The head-width-64 kernels on inputs where each head carries one head-width-4 head of the spec's shape in its
    dimensions desloc .. desloc + 3 (tests/reducoes.py, family 1; from 32 on in the head's second block, the first
    all-zero) give that head's outputs as the oracle's head-width-4 code computes them -- the code the
    reference's goldens pin (ops.py:186-258): P, o, and the backward's gq, gk, gv."""
    import reducoes as RD
    Bt, T = 2, 128
    (q4, g4), (q64, g64) = RD.problemas(5151 + desloc, Bt, T, desloc)
    cpu = CPU(32)
    gpu = GPU(32, vigiar=True)
    Q4, G4 = (tuple(cpu.dev(v) for v in x) for x in (q4, g4))
    Q64, G64 = (tuple(gpu.dev(v) for v in x) for x in (q64, g64))
    old_c, old_g = cpu.limite(limite), gpu.limite(limite)
    try:
        f4 = cpu.ops.atencao(Q4, Bt, T, RD.H4)
        f64 = gpu.ops.atencao(Q64, Bt, T, RD.H64)
        b4 = cpu.ops.atencao_back(G4, Q4, f4[1], Bt, T, RD.H4)
        b64 = gpu.ops.atencao_back(G64, Q64, f64[1], Bt, T, RD.H64)
    finally:
        cpu.limite(old_c)
        gpu.limite(old_g)
    RD.confere_frente([[host(x) for x in f4[0]], host(f4[1])], [[host(x) for x in f64[0]], host(f64[1])], Bt, desloc)
    RD.confere_tras([host(x) for x in b4], [host(x) for x in b64], desloc)
