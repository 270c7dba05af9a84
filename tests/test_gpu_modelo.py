"""Model-level parity of the HIP path.

* two full training steps (522 ops each: forward, backward, optimizer) at the reference model shape
  (V=256, D=256, H=64, FF=1024, L=12, T=128, BLK=128) at Bt=8 and Bt=16: every op output equals the spec's
  (traces written from OpsRef + Modelo.passo, the reference's `conferir 2` protocol, treino_cuda.py:48-60);
* the hipGraph-captured step replays to the same bits as eager steps, for every replay, with eager work and
  synchronization between replays; and the per-step (d_alvo, soma) of the golden loss trace;
* the fused optimizer (momento + peso of all 50 tensors in one launch, or in the epilogue of the grouped
  weight-gradient GEMMs) leaves weights, momenta and residuals bit-identical to momento then peso per tensor, with
  and without error feedback;
* a token outside the vocabulary inside a replayed graph raises ErroJatai naming op embed, scope
  "forward / embedding", row 401, value 300 (the reference's teste_erro_grafo.py:13-30).
"""
import numpy as np
import pytest
import torch

import recipe as R
import traco as TR
from backends import LOGS, host

pytestmark = pytest.mark.gpu


def _ops(vigiar=False):
    from jatai_amd import ops as O
    from jatai_amd.registro import Registro
    O.BLK = 128
    reg = Registro(LOGS, "modelo", vigiar=vigiar, eco=False)
    return O.OpsHip(reg), reg


@pytest.mark.parametrize("nome", TR.TRACOS)
def test_dois_passos_vs_spec(nome):
    ops, reg = _ops()
    reg.novo_passo(0)
    _, init, passos = TR.roda(ops, reg, "cuda", 2, host, nome)
    reg.fim_passo()
    TR.confere(init, passos, nome)


def _estado(m):
    return [R.sha(host(t)) for n in m.p for t in (*m.p[n], *m.mom[n], *m.res[n])]


@pytest.mark.parametrize("nome", TR.TRACOS)
def test_grafo_igual_ao_eager_e_ao_spec(nome):
    from jatai_amd.modelo import Modelo, PassoGravado
    g = TR.gold(nome)
    f = g["forma"]
    n = len(g["passos"])                                 # every step of the golden loss trace
    ops, reg = _ops()
    dev = "cuda"
    mk = lambda: Modelo(f["V"], f["D"], f["H"], f["FF"], f["L"], f["semente"], dev, ops, reg)
    eager, grafado = mk(), mk()
    for m in (eager, grafado):
        m.perda_inteira = True
    hist_e, hist_g = [], []
    reg.novo_passo(0)
    for p in range(n):
        tok, alvo = TR.lote(p, f["Bt"], f["T"], f["V"], dev)
        d, s = eager.passo(tok, alvo, k_lr=f["k_lr"])
        hist_e.append((R.sha(host(d)), R.sha(host(s))))
    reg.fim_passo()
    tok, alvo = TR.lote(0, f["Bt"], f["T"], f["V"], dev)
    d, s = grafado.passo(tok, alvo, k_lr=f["k_lr"])
    hist_g.append((R.sha(host(d)), R.sha(host(s))))
    grafado.perda_inteira = False
    pg = PassoGravado(grafado, f["Bt"], f["T"], f["k_lr"])
    perdas = []
    for p in range(1, n):
        reg.novo_passo(p)
        tok, alvo = TR.lote(p, f["Bt"], f["T"], f["V"], dev)
        perdas.append(float(pg(tok, alvo)))
        torch.cuda.synchronize()
        hist_g.append((R.sha(host(pg.d_alvo)), R.sha(host(pg.soma))))
        reg.fim_passo()
        _ = torch.ones(1024, device=dev).sum().item()        # eager work between replays
    assert hist_g == hist_e, "graph replays differ from eager steps"
    assert _estado(grafado) == _estado(eager), "weights / momentum / residuals differ after graph replays"
    for p in range(n):
        assert [hist_e[p][0], hist_e[p][1]] == [g["passos"][p]["d_alvo"], g["passos"][p]["soma"]], f"step {p} vs spec"
    for p, x in enumerate(perdas, start=1):
        assert abs(x - g["passos"][p]["perda"]) <= 1e-12 * abs(g["passos"][p]["perda"])


def test_erro_no_grafo():
    from jatai_amd.modelo import Modelo, PassoGravado
    from jatai_amd.registro import ErroJatai
    g = TR.gold()
    f = g["forma"]
    ops, reg = _ops()
    m = Modelo(f["V"], f["D"], f["H"], f["FF"], 2, 0, "cuda", ops, reg)
    tok, alvo = TR.lote(0, 8, 128, 256, "cuda")
    reg.novo_passo(0); m.passo(tok, alvo, k_lr=4); reg.fim_passo()
    pg = PassoGravado(m, 8, 128, 4)
    reg.novo_passo(1); pg(tok, alvo); reg.fim_passo()
    ruim = tok.clone()
    ruim[3, 17] = 300
    reg.novo_passo(2)
    with pytest.raises(ErroJatai) as e:
        pg(ruim, alvo)
        reg.fim_passo()
    msg = str(e.value)
    assert "forward / embedding" in msg and "linha 401, coluna 0" in msg and "valor    : 300" in msg, msg
    assert "operacao : embed" in msg
    # the inputs of the failing launch were saved (registro.py's contract with jatai_cuda/registro.py:126-130):
    # the embedding weights as the graph holds them and the replay's tokens, which reproduce the event on the CPU
    ev = reg.ultimo_evento
    assert ev.lancamento.op == "embed" and ev.idx == 401 * 256 and ev.valor == 300 and ev.arquivo in msg
    salvo = torch.load(ev.arquivo, weights_only=True)
    assert set(salvo) == {"W", "tok"}
    assert torch.equal(salvo["W"], m.p["emb"][0].cpu())
    assert int(salvo["tok"].reshape(-1)[401]) == 300 and torch.equal(salvo["tok"].reshape(-1).long(), ruim.reshape(-1).cpu())
    from oracle.ops_oracle import OpsOraculo
    W = (salvo["W"], m.p["emb"][1].cpu())
    with pytest.raises(IndexError, match="1 tokens outside the vocabulary of 256"):
        OpsOraculo(128).embed(W, salvo["tok"])


@pytest.mark.parametrize("dw_lote,compacto", [(True, True), (False, True), (False, False)],
                         ids=["otimizador-no-gemm", "tabela", "tabela-expoente-por-valor"])
@pytest.mark.parametrize("ef", [True, False])
def test_otimizador_fundido_igual_por_tensor(ef, dw_lote, compacto):
    """The fused optimizer (one launch over the table of all tensors, reading the gradient exponents in the grouped
    GEMM's compact form or one per value; or inside the grouped GEMM's epilogue) equals momento then peso per
    tensor."""
    from jatai_amd.modelo import Modelo
    g = TR.gold()
    f = g["forma"]
    ops, reg = _ops()
    mk = lambda: Modelo(f["V"], f["D"], f["H"], f["FF"], f["L"], f["semente"], "cuda", ops, reg)
    fundido, separado = mk(), mk()
    separado.otimizador_fundido = False
    fundido.otim_no_gemm = dw_lote                  # True: momento + peso in the grouped GEMM's epilogue
    fundido.grad_compacto = compacto
    assert fundido.otimizador_fundido and fundido._otim_no_gemm() == dw_lote
    for m in (fundido, separado):
        m.error_feedback = ef
    reg.novo_passo(0)
    for p in range(3):
        tok, alvo = TR.lote(p, f["Bt"], f["T"], f["V"], "cuda")
        a = float(fundido.passo(tok, alvo, k_lr=f["k_lr"]))
        b = float(separado.passo(tok, alvo, k_lr=f["k_lr"]))
        assert a == b, (p, a, b)
    reg.fim_passo()
    assert _estado(fundido) == _estado(separado)
    if not dw_lote:
        assert fundido._gbuf_compacto == compacto
