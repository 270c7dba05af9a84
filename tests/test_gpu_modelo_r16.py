"""The config-5 architecture at test scale: the training step with the 16-bit residual stream (R16: para16 /
soma16 / para8 carry the residual, modelo.py:60-130) at the BASELINE widths (D=512, 8 heads x 64, FF=2048, V=256,
T=256, BLK=32), with 2 layers and 2 sequences. Every op output of the HIP path equals the CPU oracle's; the fused
step (batched transposes, grouped weight-gradient GEMMs, fused optimizer, the residual adds with their INT8 copies
in the GEMM and rms_back launches) leaves the same weights, momenta and
residuals; a third step replayed from a captured hipGraph equals the eager op-by-op step.

The R16 ops have no counterpart in the reference's spec (their oracle restates the CUDA kernels,
jatai_cuda.cu:446-531), so this composition is pinned by the oracle alone."""
import pytest
import torch

import cases as CS
import recipe as R
from backends import LOGS, host

pytestmark = pytest.mark.gpu


def test_passo_r16_vs_oraculo():
    from jatai_amd import ops as O
    from jatai_amd.modelo import Modelo, PassoGravado
    from jatai_amd.registro import Registro
    from oracle.ops_oracle import OpsOraculo
    import traco as TR
    O.BLK = 32
    try:
        V, D, H, FF, L, Bt, T = 256, 512, 8, 2048, 2, 2, 256
        reg = Registro(LOGS, "modelo_r16", eco=False)
        gpu = CS.Gravador(O.OpsHip(reg), host)
        cpu = CS.Gravador(OpsOraculo(32), host)
        mg = Modelo(V, D, H, FF, L, 0, "cuda", gpu, reg, r16=True)
        mc = Modelo(V, D, H, FF, L, 0, "cpu", cpu, TR.RegStub(), r16=True)
        mg.otimizador_fundido = mg.transpostas_em_lote = mg.dw_em_lote = mg.quant_na_atencao = mg.transposta_na_gemm = mg.transposta_na_relu2 = mg.rms_soma = mg.perda_fundida = False
        mg.soma16_fundida = False
        mf = Modelo(V, D, H, FF, L, 0, "cuda", O.OpsHip(reg), reg, r16=True)
        assert mf.soma16_fundida
        for p in range(2):
            x = R.tokens(R.substream(37, f"r16 {p}"), Bt * (T + 1), V).reshape(Bt, T + 1)
            tok = torch.from_numpy(x[:, :-1].copy()).long()
            alvo = torch.from_numpy(x[:, 1:].copy()).long()
            gpu.log, cpu.log = [], []
            reg.novo_passo(p)
            pg = float(mg.passo(tok.cuda(), alvo.cuda(), k_lr=4))
            pf = float(mf.passo(tok.cuda(), alvo.cuda(), k_lr=4))
            reg.fim_passo()
            pc = float(mc.passo(tok, alvo, k_lr=4))
            assert any(op == "soma16" for op, _ in cpu.log), "the R16 path did not run"
            assert len(gpu.log) == len(cpu.log)
            for k, (a, b) in enumerate(zip(gpu.log, cpu.log)):
                assert list(a) == list(b), f"step {p}, op #{k} '{b[0]}' differs from the oracle"
            assert abs(pg - pc) <= 1e-12 * abs(pc)
            assert abs(pf - pg) <= 1e-14 * abs(pg)     # the fused model's loss sums in another order
        est = lambda m: [R.sha(host(t)) for n in m.p for t in (*m.p[n], *m.mom[n], *m.res[n])]
        assert est(mf) == est(mg), "fused R16 step differs from the op-by-op step"
        pgraf = PassoGravado(mf, Bt, T, 4)
        x = R.tokens(R.substream(37, "r16 2"), Bt * (T + 1), V).reshape(Bt, T + 1)
        tok, alvo = torch.from_numpy(x[:, :-1].copy()).long().cuda(), torch.from_numpy(x[:, 1:].copy()).long().cuda()
        reg.novo_passo(2)
        a = float(pgraf(tok, alvo))
        torch.cuda.synchronize()
        reg.fim_passo()
        b = float(mg.passo(tok, alvo, k_lr=4))
        assert abs(a - b) <= 1e-14 * abs(b)
        assert est(mf) == est(mg), "graph-replayed fused R16 step differs from the eager op-by-op step"
    finally:
        O.BLK = 128
