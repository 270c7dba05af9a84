"""Batched launches that have no reference counterpart, against the per-tensor ops they replace (bit-exact):

* transpoe_lote over 70 tensors of mixed shapes (two launches: 64 tensors per launch) equals transpoe of each,
  at BLK 32 and 128, and each result equals the CPU oracle's transpose; and so does one launch of ~8.4k tiles
  (4 tiles per workgroup, a partial last workgroup);
* the model step with batched transposes leaves weights, momenta and residuals identical to one transpoe per use;
* gemm_cru_lote over 70 GEMMs (two launches) equals one raw gemm each, at BLK 32 and 128, and a model step
  with the deferred grouped weight-gradient GEMMs equals the step with one GEMM per gradient.
"""
import numpy as np
import pytest
import torch

import recipe as R
from backends import CPU, GPU, host

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("blk", [32, 128])
def test_transpoe_lote_igual_a_transpoe(blk):
    gpu, cpu = GPU(blk, vigiar=True), CPU(blk)
    formas = [(128 * (1 + i % 4), 64 * (2 + i % 5)) for i in range(70)]
    formas = [(r, c - c % blk if c % blk else c) for r, c in formas]
    xs_h = [R.bloco(R.substream(7, f"lote {i}"), r, c, blk, espalha=6, e0=-6) for i, (r, c) in enumerate(formas)]
    xs = [tuple(gpu.dev(a) for a in x) for x in xs_h]
    lote = gpu.ops.transpoe_lote(xs)
    um = [gpu.ops.transpoe(x) for x in xs]
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(lote, um)):
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1]), f"tensor {i} {formas[i]}"
    for i in (0, 33, 69):
        ref = cpu.ops.transpoe(tuple(cpu.dev(a) for a in xs_h[i]))
        assert np.array_equal(host(lote[i][0]), host(ref[0])) and np.array_equal(host(lote[i][1]), host(ref[1]))


@pytest.mark.parametrize("blk", [32, 128])
def test_transpoe_lote_grande_igual_a_transpoe(blk):
    """64 tensors, ~8.4k tiles in one launch: the launch with 4 tiles per workgroup (from 8192 tiles), whose last
    workgroup holds a partial set of tiles (the total is not a multiple of 4)."""
    gpu, cpu = GPU(blk, vigiar=True), CPU(blk)
    formas = [(128 * (3 + i % 7), 64 * (10 + (7 * i) % 27)) for i in range(64)]
    formas = [(r, c - c % blk if c % blk else c) for r, c in formas]
    tiles = sum((r // 128) * (c // 64) for r, c in formas)
    assert tiles >= 8192 and tiles % 4 != 0
    xs_h = [R.bloco(R.substream(8, f"lote grande {i}"), r, c, blk, espalha=6, e0=-6) for i, (r, c) in enumerate(formas)]
    xs = [tuple(gpu.dev(a) for a in x) for x in xs_h]
    lote = gpu.ops.transpoe_lote(xs)
    um = [gpu.ops.transpoe(x) for x in xs]
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(lote, um)):
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1]), f"tensor {i} {formas[i]}"
    for i in (0, 31, 63):
        ref = cpu.ops.transpoe(tuple(cpu.dev(a) for a in xs_h[i]))
        assert np.array_equal(host(lote[i][0]), host(ref[0])) and np.array_equal(host(lote[i][1]), host(ref[1]))


def test_modelo_transpostas_em_lote():
    import traco as TR
    from jatai_amd import ops as O
    from jatai_amd.modelo import Modelo
    from jatai_amd.registro import Registro
    from backends import LOGS
    O.BLK = 128
    reg = Registro(LOGS, "lotes", vigiar=False, eco=False)
    ops = O.OpsHip(reg)
    f = TR.gold()["forma"]
    mk = lambda: Modelo(f["V"], f["D"], f["H"], f["FF"], f["L"], f["semente"], "cuda", ops, reg)
    a, b = mk(), mk()
    b.transpostas_em_lote = False
    assert a.transpostas_em_lote
    reg.novo_passo(0)
    for p in range(2):
        tok, alvo = TR.lote(p, f["Bt"], f["T"], f["V"], "cuda")
        assert float(a.passo(tok, alvo, k_lr=f["k_lr"])) == float(b.passo(tok, alvo, k_lr=f["k_lr"]))
    est = lambda m: [R.sha(host(t)) for n in m.p for t in (*m.p[n], *m.mom[n], *m.res[n])]
    assert est(a) == est(b)


@pytest.mark.parametrize("blk,K", [(32, 512), (128, 512), (32, 2048), (128, 2048), (32, 8192), (128, 8192)])
def test_gemm_cru_lote_igual_a_gemm(blk, K):
    """70 GEMMs in two grouped launches equal one raw gemm each: K = 512 and 2048 in one chunk of shift tables,
    K = 8192 in chunks (1024 values at BLK 32, 2048 at BLK 128)."""
    gpu = GPU(blk, vigiar=True)
    formas = [(32 * (1 + i % 5), 128 * (1 + i % 3)) for i in range(70)]
    pares, ref = [], []
    for i, (M, N) in enumerate(formas):
        A = tuple(gpu.dev(a) for a in R.bloco(R.substream(8, f"A {i}"), M, K, blk, espalha=4, e0=-6))
        B = tuple(gpu.dev(a) for a in R.bloco(R.substream(8, f"B {i}"), N, K, blk, espalha=4, e0=-9))
        pares.append((A, B, None))
        ref.append(gpu.ops.gemm(A, B, cru=True))
    out = gpu.ops.gemm_cru_lote(pares)
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(out, ref)):
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1]), f"GEMM {i} {formas[i]}"


@pytest.mark.parametrize("blk,K,bm", [(32, 2048, 0), (128, 2048, 0), (32, 8192, 0), (32, 2048, 64), (32, 2048, 128),
                                      (128, 2048, 128), (32, 8192, 128)])
def test_gemm_cru_lote_compacto(blk, K, bm):
    """gemm_cru_lote with compact exponents: the same accumulators, and exponent vectors (RA_i, then RB_j - 4) whose
    sums are the per-value exponents of the plain launch. bm = 0: ragged M (multiples of 32), so the group runs
    32-row tiles; bm = 64 / 128 (jt_gemm_bm): every M a multiple of 128, so the group runs 64- or 128-row tiles and
    the compact epilogue writes RA for 64 or 128 rows per tile."""
    gpu = GPU(blk, vigiar=True)
    if bm == 0:
        formas = [(32 * (1 + i % 5), 128 * (1 + i % 3)) for i in range(20)] + [(512, 2048), (2048, 512)]
    else:
        formas = [(128 * (1 + i % 4), 128 * (1 + i % 3)) for i in range(12)] + [(512, 2048), (2048, 512)]
    pares = []
    for i, (M, N) in enumerate(formas):
        A = tuple(gpu.dev(a) for a in R.bloco(R.substream(9, f"A {i}"), M, K, blk, espalha=5, e0=-6))
        B = tuple(gpu.dev(a) for a in R.bloco(R.substream(9, f"B {i}"), N, K, blk, espalha=5, e0=-9))
        pares.append((A, B))
    try:
        gpu.ops.lib.jt_gemm_bm(bm)
        cheio = gpu.ops.gemm_cru_lote([(A, B, None) for A, B in pares])
        comp = gpu.ops.gemm_cru_lote([(A, B, None) for A, B in pares], compacto=True)
        torch.cuda.synchronize()
    finally:
        gpu.ops.lib.jt_gemm_bm(0)
    ref = [gpu.ops.gemm(A, B, cru=True) for A, B in pares]          # the single-GEMM path at the automatic tile
    for i, (a, b) in enumerate(zip(cheio, ref)):
        assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1]), f"GEMM {i} {formas[i]}: grouped vs single"
    for i, ((M, N), a, b) in enumerate(zip(formas, cheio, comp)):
        assert tuple(b[1].shape) == (M + N,)
        assert torch.equal(a[0], b[0]), f"GEMM {i} {formas[i]}: accumulators"
        e = b[1][:M].long()[:, None] + b[1][M:].long()[None, :]
        assert torch.equal(a[1].long(), e.clamp(min=-30000)), f"GEMM {i} {formas[i]}: exponents"


def test_modelo_dw_em_lote():
    import traco as TR
    from jatai_amd import ops as O
    from jatai_amd.modelo import Modelo
    from jatai_amd.registro import Registro
    from backends import LOGS
    O.BLK = 128
    reg = Registro(LOGS, "lotes", vigiar=False, eco=False)
    ops = O.OpsHip(reg)
    f = TR.gold()["forma"]
    mk = lambda: Modelo(f["V"], f["D"], f["H"], f["FF"], f["L"], f["semente"], "cuda", ops, reg)
    a, b = mk(), mk()
    b.dw_em_lote = False
    assert a.dw_em_lote
    reg.novo_passo(0)
    for p in range(2):
        tok, alvo = TR.lote(p, f["Bt"], f["T"], f["V"], "cuda")
        assert float(a.passo(tok, alvo, k_lr=f["k_lr"])) == float(b.passo(tok, alvo, k_lr=f["k_lr"]))
    est = lambda m: [R.sha(host(t)) for n in m.p for t in (*m.p[n], *m.mom[n], *m.res[n])]
    assert est(a) == est(b)
