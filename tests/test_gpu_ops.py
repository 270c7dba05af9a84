"""Op-level parity of the HIP path (OpsHip -> C ABI -> gfx950 kernels) against the reference spec.

* the 40 cases of the reference op suite (jatai_cuda/teste_ops.py:57-98) at BLK 128 and 32: every output of
  every call must hash to the value the spec `OpsRef` produced (tests/golden/ops_blk*.json); on a mismatch the
  same inputs go through the CPU oracle to name the first differing element;
* BASELINE config 1 (512^3 GEMM, BLK 32 and 128) against its golden hashes;
* config 2 and 3 shapes (M = 2048, D = 512, FF = 2048, V = 256, BLK = 32) against the CPU oracle, bit-exact;
* split-K: the raw GEMM gives the same bits at every split count.
"""
import json
import os

import numpy as np
import pytest
import torch

import cases as CS
import recipe as R
from backends import CPU, GPU, host, primeira_diferenca

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CASOS = CS.casos()


def _gold(nome):
    return json.load(open(os.path.join(GOLD, nome)))


def _roda(be, i, blk):
    nome, fn = CASOS[i]
    rec = CS.Gravador(be.ops, host)
    g = CS.Gen(R.substream(1000 + i, nome), blk, be.dev)
    saida = fn(rec, g, be)
    return rec.log, saida


@pytest.mark.parametrize("blk", [128, 32])
@pytest.mark.parametrize("i", range(len(CASOS)), ids=[n for n, _ in CASOS])
def test_caso_vs_spec(blk, i):
    gold = _gold(f"ops_blk{blk}.json")[i]
    gpu = GPU(blk, vigiar=True)
    log, saida = _roda(gpu, i, blk)
    torch.cuda.synchronize()
    esperado = [list(x) for x in gold["chamadas"]]
    obtido = [list(x) for x in log]
    if obtido != esperado:
        _, ref = _roda(CPU(blk), i, blk)
        difs = [primeira_diferenca(host(a), host(b)) for a, b in zip(CS.plano(saida), CS.plano(ref))]
        pytest.fail(f"{CASOS[i][0]} (BLK={blk}) differs from the spec; first difference per output vs the oracle "
                    f"(flat index, gpu, oracle, count): {difs}")


GEMMS = [i for i, (n, _) in enumerate(CASOS) if n.startswith("gemm")]


@pytest.fixture
def tile_gemm(request):
    """jt_gemm_bm(bm) for the test, then back to the automatic tile (the reference's tile() helper,
    teste_ops.py:34-40)."""
    from jatai_amd import ops as O
    lib = O.carrega_lib()
    lib.jt_gemm_bm(request.param)
    yield request.param
    lib.jt_gemm_bm(0)


@pytest.mark.parametrize("tile_gemm", [64, 128], indirect=True)
@pytest.mark.parametrize("blk", [128, 32])
@pytest.mark.parametrize("i", GEMMS, ids=[CASOS[i][0] for i in GEMMS])
def test_caso_gemm_tile_forcado(blk, i, tile_gemm):
    """Every GEMM case of the reference suite again with the taller tiles forced through jt_gemm_bm (64 and 128
    rows: 8 and 16 waves per K-split group), as teste_ops.py:99-103 runs each GEMM at both of its tiles: the same
    hashes as the spec's."""
    test_caso_vs_spec(blk, i)


@pytest.mark.parametrize("tile_gemm", [64, 128], indirect=True)
def test_gemm_tile_forcado_k_longo_e_lote(tile_gemm):
    """Taller tiles on the long-K path (K = 8192: four 2048-value chunks of shift tables), on the transposed
    ReLU^2-backward copy (two blocks per column of the tile at 64 rows, four at 128) and on a grouped launch, each
    equal to the oracle (or to the separate launches)."""
    blk = 32
    gpu, cpu = GPU(blk), CPU(blk)
    s = lambda t: R.substream(78, f"{t} {tile_gemm}")
    for M, N, K in ((128, 256, 8192), (256, 384, 1024)):
        A = R.bloco(s(f"A{K}"), M, K, blk, espalha=5, e0=-8)
        B = R.bloco(s(f"B{K}"), N, K, blk, espalha=5, e0=-12)
        X = R.bloco(s(f"X{K}"), M, N, blk, espalha=3, e0=2)
        ref = [CS.plano(t) for t in _gemm_modos(cpu.ops, *[tuple(cpu.dev(v) for v in T) for T in (A, B, X)])]
        out = [CS.plano(t) for t in _gemm_modos(gpu.ops, *[tuple(gpu.dev(v) for v in T) for T in (A, B, X)])]
        gpu.reg.confere_device()
        for modo, (a, b) in enumerate(zip(out, ref)):
            for x, y in zip(a, b):
                assert np.array_equal(host(x), host(y)), f"K={K} mode {modo}: {primeira_diferenca(host(x), host(y))}"
        Ag, Bg, Xg = (tuple(gpu.dev(v) for v in T) for T in (A, B, X))
        Gt, GtT = gpu.ops.gemm_relu2_back_t(Ag, Bg, Xg)
        refT = cpu.ops.transpoe(cpu.ops.gemm_relu2_back(*[tuple(cpu.dev(v) for v in T) for T in (A, B, X)]))
        for x, y in zip(GtT, refT):
            assert np.array_equal(host(x), host(y)), f"K={K} transposed relu2_back: {primeira_diferenca(host(x), host(y))}"
    pares = [(tuple(gpu.dev(v) for v in R.bloco(s(f"lA{j}"), M, 1024, blk, espalha=6, e0=-20)),
              tuple(gpu.dev(v) for v in R.bloco(s(f"lB{j}"), N, 1024, blk, espalha=4, e0=-6)), None)
             for j, (M, N) in enumerate(((256, 512), (512, 128), (128, 256)))]
    lote = gpu.ops.gemm_cru_lote(pares)
    for (A, B, _), G in zip(pares, lote):
        ref = gpu.ops.gemm(A, B, cru=True)
        for x, y in zip(G, ref):
            assert np.array_equal(host(x), host(y))


ATENCAO4 = [i for i, (n, _) in enumerate(CASOS) if n.startswith("atencao")]


@pytest.mark.parametrize("linhas", [1, 2])
@pytest.mark.parametrize("blk", [128, 32])
@pytest.mark.parametrize("i", ATENCAO4, ids=[CASOS[i][0] for i in ATENCAO4])
def test_caso_atencao_duas_linhas(blk, i, linhas):
    """The reference suite's attention cases with the layouts jt_atencao_linhas forces (jatai_cuda.cu:1091): one
    query row per thread, and two (rows i and T - 1 - i); the default runs 8 lanes per row. The spec's hashes."""
    from jatai_amd import ops as O
    lib = O.carrega_lib()
    lib.jt_atencao_linhas(linhas)
    try:
        test_caso_vs_spec(blk, i)
    finally:
        lib.jt_atencao_linhas(0)


DOMINIO = CS.casos_dominio()


@pytest.mark.parametrize("linhas", [0, 1, 2])
@pytest.mark.parametrize("blk", [128, 32])
@pytest.mark.parametrize("i", range(len(DOMINIO)), ids=[n for n, _ in DOMINIO])
def test_dominio_vs_spec(blk, i, linhas):
    """The rest of the reference's shape domain (rms widths 384-896, softmax V = 384 / 640, head-width-4 attention
    at H = 32 and T = 32 / 96) against the spec's hashes (tests/golden/ops_dominio_blk*.json)."""
    gold = _gold(f"ops_dominio_blk{blk}.json")[i]
    nome, fn = DOMINIO[i]
    from jatai_amd import ops as O
    lib = O.carrega_lib()
    lib.jt_atencao_linhas(linhas)
    try:
        gpu = GPU(blk, vigiar=True)
        rec = CS.Gravador(gpu.ops, host)
        saida = fn(rec, CS.Gen(R.substream(1000 + i, nome), blk, gpu.dev), gpu)
        torch.cuda.synchronize()
    finally:
        lib.jt_atencao_linhas(0)
    if [list(x) for x in rec.log] != [list(x) for x in gold["chamadas"]]:
        cpu = CPU(blk)
        ref = fn(cpu.ops, CS.Gen(R.substream(1000 + i, nome), blk, cpu.dev), cpu)
        difs = [primeira_diferenca(host(a), host(b)) for a, b in zip(CS.plano(saida), CS.plano(ref))]
        pytest.fail(f"{nome} (BLK={blk}) differs from the spec; first difference per output vs the oracle: {difs}")


@pytest.mark.parametrize("linhas", [0, 1, 2])
@pytest.mark.parametrize("blk", [128, 32])
@pytest.mark.parametrize("T", [160, 192, 256])
def test_atencao4_t_longo_vs_oraculo(T, blk, linhas):
    """Head-width-4 attention past the spec's T <= 128 (this library accepts T % 32 up to 256), forward and both
    backward variants, against the oracle: the only change from the spec there is dS's width (12 - max(0,
    ceil(log2 T) - 7) bits: 11 at T = 160 .. 256)."""
    from jatai_amd import ops as O
    Bt, H = 2, 64
    D = 4 * H
    seed = R.substream(557, f"a4 {T} {blk}")
    qn = R.bloco(R.substream(seed, "qkv"), Bt * T, 3 * D, blk, espalha=6, e0=-6, zera=0.05)
    gn = R.bloco(R.substream(seed, "go"), Bt * T, D, blk, espalha=6, e0=-20, zera=0.05)
    lib = O.carrega_lib()
    res = {}
    for nome, be in (("gpu", GPU(blk, vigiar=True)), ("cpu", CPU(blk))):
        qkv = tuple(be.dev(v) for v in qn)
        go = tuple(be.dev(v) for v in gn)
        if nome == "gpu":
            lib.jt_atencao_linhas(linhas)
        try:
            (oacc, oe), P = be.ops.atencao(qkv, Bt, T, H)
            saida = [oacc, oe, P]
            for lim in (False, True):
                old = be.limite(lim)
                try:
                    saida += list(be.ops.atencao_back(go, qkv, P, Bt, T, H))
                finally:
                    be.limite(old)
        finally:
            lib.jt_atencao_linhas(0)
        res[nome] = [host(x) for x in saida]
    for nome, a, b in zip(("oacc", "oe", "P", "gacc", "ge", "gacc limite", "ge limite"), res["gpu"], res["cpu"]):
        d = primeira_diferenca(a, b)
        assert d is None, f"T={T} {nome}: (flat index, gpu, oracle, count) = {d}"


@pytest.mark.parametrize("blk", [32, 128])
def test_de_f32_vs_oraculo(blk):
    """The fp32 data path: de_f32 on the GPU (frexp split, then jt_quant) equals the oracle's, bit for bit, on
    N(0, 1) values with zero blocks, subnormals and large values mixed in."""
    x = R.normal32(402, (256, 1024))
    x[0, :blk] = 0.0
    x[1, :4] = np.array([1e-40, -3e-39, 2.5e-45, 7.0], np.float32)
    x[2, :blk] *= np.float32(2.0 ** 60)
    res = [be.ops.de_f32(be.dev(x)) for be in (GPU(blk), CPU(blk))]
    for nome, a, b in zip(("m", "E"), *res):
        d = primeira_diferenca(host(a), host(b))
        assert d is None, f"de_f32 {nome}: {d}"


@pytest.mark.parametrize("blk", [32, 128])
def test_config1(blk):
    gold = _gold("config1.json")[str(blk)]
    gpu = GPU(blk)
    A = tuple(gpu.dev(x) for x in R.bloco(R.substream(0, "A"), 512, 512, blk, espalha=4, e0=-4))
    B = tuple(gpu.dev(x) for x in R.bloco(R.substream(0, "B"), 512, 512, blk, espalha=4, e0=-4))
    assert [R.sha(host(t)) for t in gpu.ops.gemm(A, B)] == gold["bloco"]
    assert [R.sha(host(t)) for t in gpu.ops.gemm(A, B, cru=True)] == gold["cru"]


def _compara(gpu_out, cpu_out, nome):
    for k, (a, b) in enumerate(zip(CS.plano(gpu_out), CS.plano(cpu_out))):
        d = primeira_diferenca(host(a), host(b))
        assert d is None, f"{nome}: output {k} differs from the oracle (flat index, gpu, oracle, count) = {d}"


CFG3 = [(512, 1536), (512, 512), (512, 2048), (2048, 512)]


@pytest.mark.parametrize("K,N", CFG3, ids=["qkv", "out_proj", "ffn_up", "ffn_down"])
def test_config3_gemm_shapes(K, N):
    """fwd Y = X.W^T, dX = dY.(W^T)^T and dW = (dY^T).(X^T)^T (raw) at M = 2048, BLK = 32, vs the oracle. As BASELINE
    config 3 states them: weights N(0, 0.02) and activations N(0, 1) in fp32, quantized to blocks (de_f32: the exact
    frexp split, then quant); output gradients N(0, 2^-10)."""
    blk, M = 32, 2048
    gpu, cpu = GPU(blk), CPU(blk)
    seed = R.substream(77, f"cfg3 {K} {N}")
    Xf = R.normal32(R.substream(seed, "X"), (M, K))
    Wf = R.normal32(R.substream(seed, "W"), (N, K), 0.02)
    dYf = R.normal32(R.substream(seed, "dY"), (M, N), 2.0 ** -10)
    for be in (gpu, cpu):
        o = be.ops
        X, W, dY = (o.de_f32(be.dev(v)) for v in (Xf, Wf, dYf))
        be.res = [o.gemm(X, W), o.gemm(dY, o.transpoe(W)), o.gemm(o.transpoe(dY), o.transpoe(X), cru=True)]
    for nome, a, b in zip(("fwd", "dX", "dW"), gpu.res, cpu.res):
        _compara(a, b, f"config3 K={K} N={N} {nome}")


def test_config2_elementwise():
    """Every non-GEMM op at M = 2048, D = 512, FF = 2048, V = 256, BLK = 32, vs the oracle."""
    blk, M, D, FF, V = 32, 2048, 512, 2048, 256
    gpu, cpu = GPU(blk), CPU(blk)
    s = lambda t: R.substream(88, t)
    # activations fp32 N(0, 1) and weights fp32 N(0, 0.02) through de_f32; gradients fp32 normal
    # at their training scale; raw inputs, momentum and residual as integer recipes (jatai_cuda/teste_ops.py:18-31)
    flut = dict(x=R.normal32(s("x"), (M, D)), y=R.normal32(s("y"), (M, D)), h=R.normal32(s("h"), (M, FF)),
                g=R.normal32(s("g"), (M, D), 2.0 ** -12), gh=R.normal32(s("gh"), (M, FF), 2.0 ** -16),
                w=R.normal32(s("w"), (D, FF), 0.02))
    ins = dict(c=R.cru(s("c"), M, D, bits=24, e0=-30), lg=R.cru(s("lg"), M, V, bits=22, e0=-20),
               mom=R.bloco(s("mom"), D, FF, blk, e0=-15), res=R.bloco(s("res"), D, FF, blk, e0=-20, zera=0.3),
               gw=R.cru(s("gw"), D, FF, bits=28, e0=-50))
    alvo = R.tokens(s("alvo"), M, V)
    for be in (gpu, cpu):
        o = be.ops
        d = {k: tuple(be.dev(v) for v in t) for k, t in ins.items()}
        d.update({k: o.de_f32(be.dev(v)) for k, v in flut.items()})
        Y, cache = o.rms(d["x"])
        w = tuple(t.clone() for t in d["w"])
        mom = tuple(t.clone() for t in d["mom"])
        res = tuple(t.clone() for t in d["res"])
        o.momento(d["gw"], mom)
        o.peso(w, mom, res, 4, True)
        be.res = [Y, cache, o.rms_back(d["g"], Y, cache), o.soma(d["x"], d["y"]), o.relu2(d["h"]), o.relu2_back(d["gh"], d["h"]),
                  o.quant(d["c"]), o.softmax_ce(d["lg"], be.dev(alvo)), o.transpoe(d["h"]), mom, w, res,
                  o.para8(o.soma16(o.para16(d["x"]), d["y"])),
                  o.gemm_soma(d["x"], _wsq(be, blk), d["y"])]
    nomes = ["rms", "rms cache", "rms_back", "soma", "relu2", "relu2_back", "quant", "softmax_ce", "transpoe", "momento",
             "peso W", "peso R", "R16 trio", "gemm_soma"]
    for nome, a, b in zip(nomes, gpu.res, cpu.res):
        _compara(a, b, f"config2 {nome}")


def _wsq(be, blk):
    return tuple(be.dev(v) for v in R.bloco(R.substream(89, "wsq"), 512, 512, blk, espalha=2, e0=-12))


def test_split_k_same_bits():
    """Raw dW GEMM (K = tokens) gives identical bits with split-K forced off and at the default target."""
    blk = 32
    gpu = GPU(blk)
    A = tuple(gpu.dev(v) for v in R.bloco(5, 512, 2048, blk, espalha=6))
    B = tuple(gpu.dev(v) for v in R.bloco(6, 256, 2048, blk, espalha=6))
    base = [host(t) for t in gpu.ops.gemm(A, B, cru=True)]
    for alvo in (1, 64, 4096):
        gpu.ops.lib.jt_gemm_split(alvo)
        try:
            out = [host(t) for t in gpu.ops.gemm(A, B, cru=True)]
        finally:
            gpu.ops.lib.jt_gemm_split(1024)
        assert all(np.array_equal(a, b) for a, b in zip(base, out)), f"split target {alvo}"


@pytest.mark.parametrize("blk,K", [(32, 32), (32, 96), (32, 160), (32, 1376), (128, 128), (128, 384)])
def test_gemm_k_impar_todos_os_modos(blk, K):
    """K-block counts that leave a partial last stage (odd at BLK=32) and K = one block: the five GEMM modes, at
    split targets that select 1, 2 and 4 K-splits, vs the oracle."""
    M, N = 256, 256
    gpu, cpu = GPU(blk), CPU(blk)
    s = lambda t: R.substream(91, f"{blk} {K} {t}")
    An = R.bloco(s("A"), M, K, blk, espalha=4, e0=-6)
    Bn = R.bloco(s("B"), N, K, blk, espalha=4, e0=-9)
    Xn = R.bloco(s("X"), M, N, blk, espalha=3, e0=-4)
    res = {}
    for nome, be in (("cpu", cpu), ("gpu", gpu)):
        A, B, X = (tuple(be.dev(v) for v in t) for t in (An, Bn, Xn))
        o = be.ops
        res[nome] = lambda o=o, A=A, B=B, X=X: [o.gemm(A, B), o.gemm(A, B, cru=True), o.gemm_soma(A, B, X),
                                                 o.gemm_relu2(A, B), o.gemm_relu2_back(A, B, X)]
    ref = res["cpu"]()
    for alvo in (1, 64, 1024):
        gpu.ops.lib.jt_gemm_split(alvo)
        try:
            out = res["gpu"]()
        finally:
            gpu.ops.lib.jt_gemm_split(1024)
        for modo, (a, b) in enumerate(zip(out, ref)):
            _compara(a, b, f"BLK={blk} K={K} mode {modo} split target {alvo}")


@pytest.mark.parametrize("M,N,K", [(2048, 2048, 512), (256, 384, 96), (64, 128, 32)])
def test_gemm_relu2_back_t(M, N, K):
    """Mode 4 with the transposed copy (BLK = 32): the block output equals gemm_relu2_back and the copy equals
    transpoe of it."""
    blk = 32
    gpu = GPU(blk, vigiar=True)
    s = lambda t: R.substream(92, f"{M} {N} {K} {t}")
    A = tuple(gpu.dev(v) for v in R.bloco(s("A"), M, K, blk, espalha=4, e0=-6))
    B = tuple(gpu.dev(v) for v in R.bloco(s("B"), N, K, blk, espalha=4, e0=-9))
    Hh = tuple(gpu.dev(v) for v in R.bloco(s("H"), M, N, blk, espalha=3, e0=-4, zera=0.1))
    o = gpu.ops
    G, Gt = o.gemm_relu2_back_t(A, B, Hh)
    ref = o.gemm_relu2_back(A, B, Hh)
    reft = o.transpoe(ref) if M % 128 == 0 else None
    _compara(G, ref, "gemm_relu2_back")
    if reft is not None:
        _compara(Gt, reft, "transpoe")
    else:                                                            # transpoe needs R % 128: check against the oracle
        cpu = CPU(blk)
        _compara(Gt, cpu.ops.transpoe(tuple(torch.from_numpy(host(t)) for t in ref)), "transpoe (oracle)")


@pytest.mark.parametrize("M,N,K,bm", [(2048, 2048, 512, 0), (256, 384, 96, 0), (64, 128, 32, 0), (512, 1024, 1536, 64),
                                      (512, 512, 4096, 32)])
def test_gemm_relu2_t(M, N, K, bm):
    """Mode 3 with the transposed copy of its ReLU^2 output (BLK = 32): h and a equal gemm_relu2's and the copy
    equals transpoe(a), at the automatic tile (128 rows at config 4's shape) and at forced 64- and 32-row tiles."""
    blk = 32
    gpu = GPU(blk, vigiar=True)
    s = lambda t: R.substream(96, f"{M} {N} {K} {t}")
    A = tuple(gpu.dev(v) for v in R.bloco(s("A"), M, K, blk, espalha=4, e0=-6, zera=0.05))
    B = tuple(gpu.dev(v) for v in R.bloco(s("B"), N, K, blk, espalha=4, e0=-9))
    o = gpu.ops
    try:
        o.lib.jt_gemm_bm(bm)
        h, a, at = o.gemm_relu2_t(A, B)
    finally:
        o.lib.jt_gemm_bm(0)
    hr, ar = o.gemm_relu2(A, B)
    _compara(h, hr, "gemm_relu2: h")
    _compara(a, ar, "gemm_relu2: a")
    if M % 128 == 0:
        _compara(at, o.transpoe(ar), "transpoe")
    else:                                                            # transpoe needs R % 128: check against the oracle
        cpu = CPU(blk)
        _compara(at, cpu.ops.transpoe(tuple(torch.from_numpy(host(t)) for t in ar)), "transpoe (oracle)")


@pytest.mark.parametrize("blk,D", [(32, 512), (128, 256), (32, 1024)])
def test_rms_back_soma(blk, D):
    """soma(x, rms_back(g, y, cache)) in one launch equals the two ops."""
    gpu = GPU(blk, vigiar=True)
    M = 512
    s = lambda t: R.substream(93, f"{blk} {D} {t}")
    X0 = tuple(gpu.dev(v) for v in R.bloco(s("x0"), M, D, blk, espalha=3, e0=-6))
    G = tuple(gpu.dev(v) for v in R.bloco(s("g"), M, D, blk, espalha=4, e0=-20))
    X = tuple(gpu.dev(v) for v in R.bloco(s("x"), M, D, blk, espalha=3, e0=-18, zera=0.05))
    o = gpu.ops
    Y, cache = o.rms(X0)
    _compara(o.rms_back_soma(G, Y, cache, X), o.soma(X, o.rms_back(G, Y, cache)), "rms_back_soma")


@pytest.mark.parametrize("blk,M,N,K,alvo,bm", [(32, 512, 512, 512, 1024, 0), (32, 512, 512, 512, 1, 0), (32, 256, 512, 2048, 1024, 128),
                                                 (128, 256, 256, 512, 1024, 0), (32, 2048, 512, 1536, 1024, 64)])
def test_gemm_soma16(blk, M, N, K, alvo, bm):
    """soma16(x16, gemm(A, B)) and para8 of the sum in one launch (the R16 step's residual add) equal gemm, soma16
    and para8 in turn, at one and two K-splits and at forced tiles of 64 and 128 rows; zero blocks on both sides."""
    gpu = GPU(blk, vigiar=True)
    s = lambda t: R.substream(94, f"{blk} {M} {N} {K} {t}")
    A = tuple(gpu.dev(v) for v in R.bloco(s("A"), M, K, blk, espalha=4, e0=-6, zera=0.05))
    B = tuple(gpu.dev(v) for v in R.bloco(s("B"), N, K, blk, espalha=4, e0=-9))
    X0 = tuple(gpu.dev(v) for v in R.bloco(s("x0"), M, N, blk, espalha=3, e0=-4, zera=0.05))
    Y0 = tuple(gpu.dev(v) for v in R.bloco(s("y0"), M, N, blk, espalha=3, e0=-12, zera=0.05))
    o = gpu.ops
    X16 = o.soma16(o.para16(X0), Y0)                                 # 15-bit mantissas, zero blocks included
    try:
        gpu.ops.lib.jt_gemm_split(alvo)
        gpu.ops.lib.jt_gemm_bm(bm)
        Z, Y8 = o.gemm_soma16(A, B, X16)
        Zr = o.soma16(X16, o.gemm(A, B))
    finally:
        gpu.ops.lib.jt_gemm_split(1024)
        gpu.ops.lib.jt_gemm_bm(0)
    _compara(Z, Zr, "gemm_soma16: soma16")
    _compara(Y8, o.para8(Zr), "gemm_soma16: para8")


@pytest.mark.parametrize("blk,D", [(32, 512), (128, 256), (32, 768)])
def test_rms_back_soma16(blk, D):
    """soma16(x16, rms_back(g, y, cache)) and para8 of the sum in one launch (the R16 backward's residual update)
    equal rms_back, soma16 and para8 in turn, also at a width that is not a power of two."""
    gpu = GPU(blk, vigiar=True)
    M = 512
    s = lambda t: R.substream(95, f"{blk} {D} {t}")
    X0 = tuple(gpu.dev(v) for v in R.bloco(s("x0"), M, D, blk, espalha=3, e0=-6))
    G = tuple(gpu.dev(v) for v in R.bloco(s("g"), M, D, blk, espalha=4, e0=-20))
    X1 = tuple(gpu.dev(v) for v in R.bloco(s("x1"), M, D, blk, espalha=3, e0=-18, zera=0.05))
    Y1 = tuple(gpu.dev(v) for v in R.bloco(s("y1"), M, D, blk, espalha=3, e0=-26, zera=0.05))
    o = gpu.ops
    Y, cache = o.rms(X0)
    X16 = o.soma16(o.para16(X1), Y1)
    Z, Y8 = o.rms_back_soma16(G, Y, cache, X16)
    Zr = o.soma16(X16, o.rms_back(G, Y, cache))
    _compara(Z, Zr, "rms_back_soma16: soma16")
    _compara(Y8, o.para8(Zr), "rms_back_soma16: para8")


def test_tabela_otimizador_mantem_tensores():
    """The fused optimizer's device table keeps alive every tensor whose address it holds: built from tensors the
    caller then drops, with torch's allocator cache emptied (as entering graph capture does), the update still
    lands in those tensors and equals momento then peso on copies."""
    import gc
    blk, D, FF = 32, 512, 2048
    gpu = GPU(blk)
    s = lambda t: R.substream(91, t)
    ins = dict(w=R.bloco(s("w"), D, FF, blk, e0=-9), mom=R.bloco(s("mom"), D, FF, blk, e0=-15),
               res=R.bloco(s("res"), D, FF, blk, e0=-20, zera=0.3), gw=R.cru(s("gw"), D, FF, bits=28, e0=-50))
    d = {k: tuple(gpu.dev(v) for v in t) for k, t in ins.items()}
    w, mom, res = (tuple(t.clone() for t in d[k]) for k in ("w", "mom", "res"))
    gpu.ops.momento(d["gw"], mom)
    gpu.ops.peso(w, mom, res, 4, True)
    esperado = [R.sha(host(t)) for t in (*w, *mom, *res)]
    tab = gpu.ops.tabela_otimizador([tuple(tuple(t.clone() for t in d[k]) for k in ("gw", "mom", "w", "res"))])
    gc.collect()
    torch.cuda.empty_cache()
    gpu.ops.otimizador(tab, 4, True)
    torch.cuda.synchronize()
    assert len(tab[3]) == 8
    mom2, w2, res2 = tab[3][2:4], tab[3][4:6], tab[3][6:8]
    assert [R.sha(host(t)) for t in (*w2, *mom2, *res2)] == esperado


@pytest.mark.parametrize("compacto", [False, True])
@pytest.mark.parametrize("ef", [True, False])
def test_otimizador_t_igual_e_transpostas(ef, compacto):
    """jt_otimizador_t (one workgroup per 32 x 128 tile, writing transpoe of each new weight) leaves the same weights,
    momenta and residuals as jt_otimizador, and each transpose it writes equals transpoe of the new weight bit for bit
    (ops.py:121-123); a tensor without a transpose target is updated alike. Weight shapes of config 4 (Wqkv, Wd, out);
    the gradient exponents per value or in the grouped GEMM's compact form (row and column vectors)."""
    blk = 32
    gpu = GPU(blk)
    formas = [(1536, 512), (512, 2048), (256, 512), (512, 512)]
    itens_a, itens_b, ts = [], [], []
    for i, (M, N) in enumerate(formas):
        s = lambda t: R.substream(93, f"{i} {t}")
        w = R.bloco(s("w"), M, N, blk, espalha=4, e0=-9)
        mom = R.bloco(s("mom"), M, N, blk, e0=-15, zera=0.05)
        res = R.bloco(s("res"), M, N, blk, e0=-20, zera=0.3)
        acc, e = R.cru(s("gw"), M, N, bits=24, e0=-40)
        if compacto:                        # exponent of (i, j) = ra_i + rb_j
            ra = (-20 + R.uniform_int(s("ra"), (M,), -3, 3)).astype(np.int16)
            rb = (-24 + R.uniform_int(s("rb"), (N,), -3, 3)).astype(np.int16)
            gw = (acc, np.concatenate([ra, rb]))
        else:
            gw = (acc, e)
        a = tuple(tuple(gpu.dev(v) for v in t) for t in (gw, mom, w, res))
        b = tuple(tuple(x.clone() for x in t) for t in a)
        tw = None if i == 3 else (torch.full((N, M), 99, dtype=torch.int8, device="cuda"),
                                  torch.full((N, M // blk), 99, dtype=torch.int8, device="cuda"))
        itens_a.append(a)
        itens_b.append(b + (tw,))
        ts.append(tw)
    ta, tb = gpu.ops.tabela_otimizador(itens_a), gpu.ops.tabela_otimizador(itens_b)
    assert not ta[4] and tb[4]
    gpu.ops.otimizador(ta, 4, ef)
    gpu.ops.otimizador(tb, 4, ef)
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(itens_a, itens_b)):
        for nome, x, y in zip(("momento", "W", "residuo"), a[1:], b[1:4]):
            assert all(torch.equal(u, v) for u, v in zip(x, y)), f"tensor {i} {formas[i]}: {nome} differs"
        if ts[i] is not None:
            esperado = gpu.ops.transpoe(a[2])
            assert torch.equal(ts[i][0], esperado[0]) and torch.equal(ts[i][1], esperado[1]), f"tensor {i}: transpose differs"
        else:
            assert ts[i] is None


def _gemm_modos(ops, A, B, X):
    return [ops.gemm(A, B), ops.gemm(A, B, cru=True), ops.gemm_soma(A, B, X), ops.gemm_relu2(A, B), ops.gemm_relu2_back(A, B, X)]


@pytest.mark.parametrize("blk,K", [(32, 4608), (32, 8192), (128, 8192), (32, 16384)])
def test_gemm_k_longo_vs_oraculo(blk, K):
    """K beyond 4096 (up to 65536; the reference stops at 4096, ops.py:336-337): the kernel walks K in chunks of
    4096 with the row maxima RA, RB over all of K; every mode equals the CPU oracle, at the default K-split and
    with K-splits forced off (split target 1: one K-split) and on (split target 4096), K = 4608 leaving a short
    last chunk."""
    gpu, cpu = GPU(blk), CPU(blk)
    M, N = 64, 256
    s = lambda t: R.substream(77, f"{t} {blk} {K}")
    A = R.bloco(s("A"), M, K, blk, espalha=5, e0=-8)
    B = R.bloco(s("B"), N, K, blk, espalha=5, e0=-12)
    X = R.bloco(s("X"), M, N, blk, espalha=3, e0=2)
    ref = [CS.plano(t) for t in _gemm_modos(cpu.ops, *[tuple(cpu.dev(v) for v in T) for T in (A, B, X)])]
    for alvo in (1, 1024, 4096):
        gpu.ops.lib.jt_gemm_split(alvo)
        try:
            out = [CS.plano(t) for t in _gemm_modos(gpu.ops, *[tuple(gpu.dev(v) for v in T) for T in (A, B, X)])]
        finally:
            gpu.ops.lib.jt_gemm_split(1024)
        gpu.reg.confere_device()
        for modo, (a, b) in enumerate(zip(out, ref)):
            for x, y in zip(a, b):
                assert np.array_equal(host(x), host(y)), f"mode {modo}, split target {alvo}: {primeira_diferenca(host(x), host(y))}"


def test_gemm_cru_lote_config5_dw():
    """The weight-gradient GEMMs of a BASELINE config-5 step (K = 16384 tokens) as the step runs them: one grouped
    launch (gemm_cru_lote -> k_gemm_lote, one K-split, eight 2048-value chunks of shift tables) of the layer's five
    shapes plus the output and embedding gradients, each equal to the CPU oracle's raw GEMM (ops.py:95-108)."""
    blk, K, D, FF, V = 32, 16384, 512, 2048, 256
    gpu, cpu = GPU(blk), CPU(blk)
    formas = [("qkv", 3 * D, D), ("out-proj", D, D), ("ffn-up", FF, D), ("ffn-down", D, FF), ("out", V, D), ("emb", V, D)]
    s = lambda t: R.substream(303, t)
    ins = [(R.bloco(s(n + " dY"), M, K, blk, espalha=6, e0=-24, zera=0.02), R.bloco(s(n + " X"), N, K, blk, espalha=4, e0=-6))
           for n, M, N in formas]
    pares = [(tuple(gpu.dev(v) for v in a), tuple(gpu.dev(v) for v in b), None) for a, b in ins]
    assert gpu.ops.lib.jt_gemm_divisoes(3 * D, D, K, 1) >= 1
    out = gpu.ops.gemm_cru_lote(pares)
    gpu.reg.confere_device()
    for (n, M, N), (a, b), G in zip(formas, ins, out):
        ref = cpu.ops.gemm(tuple(cpu.dev(v) for v in a), tuple(cpu.dev(v) for v in b), cru=True)
        for x, y, parte in zip(G, ref, ("acc", "e")):
            d = primeira_diferenca(host(x), host(y))
            assert d is None, f"dW {n} [{M}x{N}, K={K}] {parte}: (flat index, gpu, oracle, count) = {d}"


def test_gemm_k_longo_acumulador_fora_do_formato():
    """K = 16384 with every mantissa 127 and one exponent: each K-block adds 16 * 32 * 127^2 (about 2^23) and the
    raw sum passes 2^30 -- past the int32 range the format allows. It is reported as a device sentinel (an
    accumulator out of range) instead of wrapping silently."""
    from jatai_amd.registro import ErroJatai
    blk, M, N, K = 32, 32, 128, 16384
    gpu = GPU(blk)
    A = (torch.full((M, K), 127, dtype=torch.int8, device="cuda"), torch.zeros(M, K // blk, dtype=torch.int8, device="cuda"))
    B = (torch.full((N, K), 127, dtype=torch.int8, device="cuda"), torch.zeros(N, K // blk, dtype=torch.int8, device="cuda"))
    gpu.ops.gemm(A, B, cru=True)
    with pytest.raises(ErroJatai, match="gemm"):
        gpu.reg.confere_device()


@pytest.mark.parametrize("blk", [32, 128])
def test_gemm_soma_estocastica(blk):
    """gemm_soma with stochastic residual rounding switched on (jt_res_estocastico(1); ops.py:308-309,
    jatai_cuda.cu:146-159 and :375): every bit equals the CPU oracle's restatement, whose seeds follow each value's
    position in the output; with the switch off again the output is the deterministic one. Spread exponents make
    the residual add drop bits in most blocks, so the hashed rounding decides many values. A captured graph follows
    the switch's value at each replay."""
    gpu, cpu = GPU(blk), CPU(blk)
    from oracle.ops_oracle import OpsOraculo
    M, N, K = 96, 384, 512
    s = lambda t: R.substream(91, f"{t} {blk}")
    A = R.bloco(s("A"), M, K, blk, espalha=5, e0=-8)
    B = R.bloco(s("B"), N, K, blk, espalha=5, e0=-12)
    X = R.bloco(s("X"), M, N, blk, espalha=4, e0=3)
    c = [tuple(cpu.dev(v) for v in T) for T in (A, B, X)]
    g = [tuple(gpu.dev(v) for v in T) for T in (A, B, X)]
    ref_est = OpsOraculo(blk, estocastico=True).gemm_soma(*c)
    ref_det = cpu.ops.gemm_soma(*c)
    assert sum(int((host(a) != host(b)).sum()) for a, b in zip(ref_est, ref_det)) > 100
    assert gpu.ops.lib.jt_res_estocastico(1) == 0
    try:
        out = gpu.ops.gemm_soma(*g)
    finally:
        gpu.ops.lib.jt_res_estocastico(0)
    det = gpu.ops.gemm_soma(*g)
    gpu.reg.confere_device()
    for x, y in zip(out, ref_est):
        assert np.array_equal(host(x), host(y)), primeira_diferenca(host(x), host(y))
    for x, y in zip(det, ref_det):
        assert np.array_equal(host(x), host(y)), primeira_diferenca(host(x), host(y))
    # as in the reference, the switch is a device global read when the kernel runs: a graph captured with it off
    # rounds stochastically on the replays made with it on
    grafo = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    try:
        with torch.cuda.graph(grafo):
            gpu.ops.lib.jt_stream(torch.cuda.current_stream().cuda_stream)
            gout = gpu.ops.gemm_soma(*g)
    finally:
        gpu.ops.lib.jt_stream(None)
    for ligado, ref in ((1, ref_est), (0, ref_det), (1, ref_est)):
        assert gpu.ops.lib.jt_res_estocastico(ligado) == 0
        try:
            grafo.replay()
            torch.cuda.synchronize()
        finally:
            gpu.ops.lib.jt_res_estocastico(0)
        for x, y in zip(gout, ref):
            assert np.array_equal(host(x), host(y)), (ligado, primeira_diferenca(host(x), host(y)))


def test_ops_conferido_sobre_hip():
    """OpsConferido (the reference's checked wrapper, ops.py:532-560) around OpsHip at BLK 32: GEMM modes, quant,
    rms and rms_back, attention forward and backward at head width 64, softmax-CE, and the in-place momento and
    peso (whose inputs the wrapper copies for the oracle before the HIP call) all agree bit for bit with the
    oracle; a mismatch would raise."""
    from jatai_amd import ops as O
    from jatai_amd.registro import Registro
    from oracle.ops_oracle import OpsConferido
    from backends import LOGS
    O.BLK = 32
    try:
        reg = Registro(LOGS, "conferido", eco=False)
        ops = OpsConferido(reg)
        s = lambda t: R.substream(93, t)
        dev = lambda T: tuple(torch.from_numpy(np.ascontiguousarray(v)).cuda() for v in T)
        A = dev(R.bloco(s("A"), 512, 512, 32, espalha=4, e0=-6))
        W = dev(R.bloco(s("W"), 1536, 512, 32, espalha=3, e0=-8))
        Wo = dev(R.bloco(s("Wo"), 512, 512, 32, espalha=3, e0=-8))
        X = dev(R.bloco(s("X"), 512, 512, 32, espalha=3, e0=1))
        n, c = ops.rms(X)
        qkv = ops.gemm(n, W)
        (oacc, oe), P = ops.atencao(qkv, 2, 256, 8)
        om = ops.quant((oacc, oe))
        x2 = ops.gemm_soma(om, Wo, X)
        h, _ = ops.gemm_relu2(x2, W)
        ops.gemm_relu2_back(x2, W, h)
        go = ops.gemm(A, Wo)
        ops.atencao_back(go, qkv, P, 2, 256, 8)
        ops.rms_back(go, n, c)
        mom = dev(R.bloco(s("M"), 512, 512, 32, espalha=2, e0=-4))
        wt = dev(R.bloco(s("Wt"), 512, 512, 32, espalha=2, e0=-6))
        res = dev(R.bloco(s("R"), 512, 512, 32, espalha=2, e0=-14))
        mom = ops.momento(ops.gemm(A, A, cru=True), mom)
        ops.peso(wt, mom, res, 4, True)
        logits = ops.gemm(A, dev(R.bloco(s("V"), 256, 512, 32, espalha=2, e0=-8)), cru=True)
        ops.softmax_ce(logits, torch.from_numpy(R.tokens(s("alvo"), 512, 256)).cuda())
        reg.lib = ops.lib
        reg.confere_device()
        assert set(ops.n) == {"rms", "gemm", "atencao", "quant", "gemm_soma", "gemm_relu2", "gemm_relu2_back", "atencao_back",
                              "rms_back", "momento", "peso", "softmax_ce"}
    finally:
        O.BLK = 128


@pytest.mark.parametrize("M", [1, 2048, 16384, 100003])
def test_perda(M):
    """The loss in one launch: against torch's float64 form on the same rows (other summation order: equal to a
    few ulps) and against the correctly rounded sum of the same float64 terms (math.fsum)."""
    import math
    gpu = GPU(32)
    rng = np.random.default_rng(M)
    d = rng.integers(0, 4096, M, dtype=np.int32)
    s = rng.integers(4096, 4096 * 256, M, dtype=np.int32)
    out = gpu.ops.perda(torch.from_numpy(d).cuda(), torch.from_numpy(s).cuda())
    x = float(out)
    ref = float((torch.from_numpy(d).double() / 256 + torch.log(torch.from_numpy(s).double() / 4096)).mean())
    exato = math.fsum(float(a) / 256 + math.log(float(b) / 4096) for a, b in zip(d, s)) / M
    assert out.dtype == torch.float64 and out.dim() == 0
    assert abs(x - ref) <= 1e-14 * abs(ref) and abs(x - exato) <= 1e-14 * abs(exato), (x, ref, exato)
