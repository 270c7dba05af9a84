"""The training step with stochastic residual rounding switched on (jt_res_estocastico(1), the JATAI_RES_EST=1
switch of ops.py:308-309; kernel text jatai_cuda.cu:146-159, :375), at the BASELINE config-4 widths with 2 layers
and 2 sequences: the fused HIP step, two steps eagerly and a third replayed from a captured hipGraph, leaves the
same losses, weights, momenta and residuals as the CPU oracle's op-by-op step with the same switch."""
import pytest
import torch

import recipe as R
from backends import LOGS, host

pytestmark = pytest.mark.gpu


def test_passo_estocastico_vs_oraculo():
    from jatai_amd import ops as O
    from jatai_amd.modelo import Modelo, PassoGravado
    from jatai_amd.registro import Registro
    from oracle.ops_oracle import OpsOraculo
    import traco as TR
    O.BLK = 32
    V, D, H, FF, L, Bt, T = 256, 512, 8, 2048, 2, 2, 256
    reg = Registro(LOGS, "modelo_est", eco=False)
    gpu = O.OpsHip(reg)
    assert gpu.lib.jt_res_estocastico(1) == 0
    try:
        mf = Modelo(V, D, H, FF, L, 0, "cuda", gpu, reg)
        mc = Modelo(V, D, H, FF, L, 0, "cpu", OpsOraculo(32, estocastico=True), TR.RegStub())
        md = Modelo(V, D, H, FF, L, 0, "cpu", OpsOraculo(32), TR.RegStub())
        est = lambda m: [R.sha(host(t)) for n in m.p for t in (*m.p[n], *m.mom[n], *m.res[n])]
        toks = []
        for p in range(3):
            x = R.tokens(R.substream(43, f"est {p}"), Bt * (T + 1), V).reshape(Bt, T + 1)
            toks.append((torch.from_numpy(x[:, :-1].copy()).long(), torch.from_numpy(x[:, 1:].copy()).long()))
        for p in range(2):
            tok, alvo = toks[p]
            reg.novo_passo(p)
            pf = float(mf.passo(tok.cuda(), alvo.cuda(), k_lr=4))
            reg.fim_passo()
            pc = float(mc.passo(tok, alvo, k_lr=4))
            assert abs(pf - pc) <= 1e-12 * abs(pc), (p, pf, pc)
            assert est(mf) == est(mc), f"step {p}: state differs from the oracle's"
        md.passo(*toks[0], k_lr=4)
        md.passo(*toks[1], k_lr=4)
        assert est(md) != est(mc), "the stochastic switch changed nothing"
        pgraf = PassoGravado(mf, Bt, T, 4)
        reg.novo_passo(2)
        a = float(pgraf(toks[2][0].cuda(), toks[2][1].cuda()))
        torch.cuda.synchronize()
        reg.fim_passo()
        b = float(mc.passo(*toks[2], k_lr=4))
        assert abs(a - b) <= 1e-12 * abs(b)
        assert est(mf) == est(mc), "graph-replayed step differs from the oracle's"
    finally:
        gpu.lib.jt_res_estocastico(0)
        O.BLK = 128
