"""One full training step at the BASELINE config-4 widths (D=512, 8 heads x 64, FF=2048, V=256, T=256, BLK=32),
with 2 layers and 2 sequences: every op output of the HIP path equals the CPU oracle's (jatai_amd.modelo.Modelo
on both backends, same init and tokens); the step with batched transposes and the fused optimizer leaves the
same weights, momenta and residuals. A third step replayed
from a captured hipGraph (fused model) equals the eager op-by-op step, and so does a fourth after a weight changed
outside the optimizer."""
import pytest
import torch

import cases as CS
import recipe as R
from backends import LOGS, host

pytestmark = pytest.mark.gpu


def test_passo_config4_vs_oraculo():
    from jatai_amd import ops as O
    from jatai_amd.modelo import Modelo
    from jatai_amd.registro import Registro
    from oracle.ops_oracle import OpsOraculo
    import traco as TR
    O.BLK = 32
    V, D, H, FF, L, Bt, T = 256, 512, 8, 2048, 2, 2, 256
    reg = Registro(LOGS, "modelo_b", eco=False)
    gpu = CS.Gravador(O.OpsHip(reg), host)
    cpu = CS.Gravador(OpsOraculo(32), host)
    mg = Modelo(V, D, H, FF, L, 0, "cuda", gpu, reg)
    mc = Modelo(V, D, H, FF, L, 0, "cpu", cpu, TR.RegStub())
    mg.otimizador_fundido = mg.transpostas_em_lote = mg.dw_em_lote = mg.quant_na_atencao = mg.transposta_na_gemm = mg.transposta_na_relu2 = mg.rms_soma = mg.perda_fundida = False   # op by op
    mf = Modelo(V, D, H, FF, L, 0, "cuda", O.OpsHip(reg), reg)  # batched transposes + fused optimizer
    assert mf.otimizador_fundido and mf.transpostas_em_lote and mf.dw_em_lote and mf.quant_na_atencao and mf.transposta_na_gemm and mf.transposta_na_relu2 and mf.rms_soma and mf.perda_fundida
    assert mf._t_na_gemm(Bt * T, FF) and mf._t_na_relu2(Bt * T, FF)   # the GEMMs' transposed writes, on by default
    mf.conversoes_salvas = True                 # and the attention backward reading the forward's conversions
    for p in range(2):
        x = R.tokens(R.substream(31, f"b4 {p}"), Bt * (T + 1), V).reshape(Bt, T + 1)
        tok = torch.from_numpy(x[:, :-1].copy()).long()
        alvo = torch.from_numpy(x[:, 1:].copy()).long()
        gpu.log, cpu.log = [], []
        reg.novo_passo(p)
        pg = float(mg.passo(tok.cuda(), alvo.cuda(), k_lr=4))
        pf = float(mf.passo(tok.cuda(), alvo.cuda(), k_lr=4))
        reg.fim_passo()
        pc = float(mc.passo(tok, alvo, k_lr=4))
        assert len(gpu.log) == len(cpu.log)
        for k, (a, b) in enumerate(zip(gpu.log, cpu.log)):
            assert list(a) == list(b), f"step {p}, op #{k} '{b[0]}' differs from the oracle"
        assert abs(pg - pc) <= 1e-12 * abs(pc)
        assert abs(pf - pg) <= 1e-14 * abs(pg)     # the fused model's loss sums in another order
    est = lambda m: [R.sha(host(t)) for n in m.p for t in (*m.p[n], *m.mom[n], *m.res[n])]
    assert est(mf) == est(mg), "fused step differs from the op-by-op step"
    # from its second step on, the fused model's backward read the weights' transposes its optimizer wrote
    assert mf.transposta_no_otimizador and mf._pt_validas
    assert not any(l.op == "transpoe" and any(x is mf.p[n][0] for x in l.entradas.values() if torch.is_tensor(x))
                   for n in mf._pt for l in reg.lancamentos), "step 2 transposed a weight again"
    # a third step: the fused model as a captured hipGraph, the op-by-op model eagerly
    from jatai_amd.modelo import PassoGravado
    pgraf = PassoGravado(mf, Bt, T, 4)
    x = R.tokens(R.substream(31, "b4 2"), Bt * (T + 1), V).reshape(Bt, T + 1)
    tok, alvo = torch.from_numpy(x[:, :-1].copy()).long().cuda(), torch.from_numpy(x[:, 1:].copy()).long().cuda()
    reg.novo_passo(2)
    a = float(pgraf(tok, alvo))
    torch.cuda.synchronize()
    reg.fim_passo()
    b = float(mg.passo(tok, alvo, k_lr=4))
    assert abs(a - b) <= 1e-14 * abs(b)
    assert est(mf) == est(mg), "graph-replayed fused step differs from the eager op-by-op step"
    # a fourth: a weight changed outside the optimizer (layer 1's out-projection copied into layer 0's) and
    # invalida_transpostas(); the graph reads the transposes its update wrote, so the replay must rewrite them first
    assert pgraf.le_transpostas
    for m in (mf, mg):
        m.p["Wo0"][0].copy_(m.p["Wo1"][0])
        m.p["Wo0"][1].copy_(m.p["Wo1"][1])
    mf.invalida_transpostas()
    x = R.tokens(R.substream(31, "b4 3"), Bt * (T + 1), V).reshape(Bt, T + 1)
    tok, alvo = torch.from_numpy(x[:, :-1].copy()).long().cuda(), torch.from_numpy(x[:, 1:].copy()).long().cuda()
    reg.novo_passo(3)
    a = float(pgraf(tok, alvo))
    torch.cuda.synchronize()
    reg.fim_passo()
    assert mf._pt_validas
    b = float(mg.passo(tok, alvo, k_lr=4))
    assert abs(a - b) <= 1e-14 * abs(b)
    assert est(mf) == est(mg), "graph step after an outside weight change differs from the eager step"
    O.BLK = 128
