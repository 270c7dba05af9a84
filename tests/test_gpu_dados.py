"""The device-resident data path: `jt_janelas` (jatai_amd.dados.Corpus) writes the same windows as the host
`lote` (treino_int8_gpu/treino.py:41-44; pinned by tests/golden/dados.json in test_dados.py) for the same generator
state; a start past the corpus end raises the device sentinel; and a graph that gathers its own windows
(PassoGravado with a corpus) trains to the same bits as one fed with the host batches."""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

import recipe as R
import traco as TR
from backends import LOGS, host

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "dados.json")


def _sha(t):
    return hashlib.sha256(np.ascontiguousarray(t.cpu().numpy().astype(np.int64)).tobytes()).hexdigest()


@pytest.fixture(scope="module")
def treino(tmp_path_factory):
    from jatai_amd import dados as DD
    p = tmp_path_factory.mktemp("corpus")
    R.corpus_sintetico(str(p))
    return DD.carregar(str(p))[0]


def _ops(vigiar=True):
    from jatai_amd import ops as O
    from jatai_amd.registro import Registro
    O.BLK = 128
    reg = Registro(LOGS, "dados", vigiar=vigiar, eco=False)
    return O.OpsHip(reg), reg


@pytest.mark.parametrize("caso", range(5))
def test_janelas_iguais_ao_lote(treino, caso):
    from jatai_amd import dados as DD
    g = json.load(open(GOLD))["lotes"][caso]
    ops, reg = _ops()
    c = DD.Corpus(ops, treino)
    g1, g2 = (torch.Generator().manual_seed(g["semente"]) for _ in range(2))
    for ref in g["passos"]:
        tok, alvo = c.lote(g1, g["Bt"], g["T"])
        x, y = DD.lote(treino, g2, g["Bt"], g["T"])
        assert tok.dtype == torch.int32 and tok.shape == (g["Bt"], g["T"])
        assert np.array_equal(host(tok), x.numpy()) and np.array_equal(host(alvo), y.numpy())
        assert _sha(tok) == ref["x"] and _sha(alvo) == ref["y"]


def test_janelas_nos_limites(treino):
    """Starts 0 and n - T - 1 (the last whole window; the reference's draw stops one short of it) are gathered;
    a start of n - T, or a negative one, raises E_ARG naming janelas and the sequence's first token, and zeroes
    that row only."""
    from jatai_amd import dados as DD
    from jatai_amd.registro import ErroJatai
    ops, reg = _ops()
    c = DD.Corpus(ops, treino)
    n, T = c.n, 64
    tok, alvo = c.janelas(torch.tensor([0, n - T - 1, 12345]), T)
    assert np.array_equal(host(tok[1]), treino[n - T - 1:n - 1].numpy()) and np.array_equal(host(alvo[1]), treino[n - T:].numpy())
    assert np.array_equal(host(tok[0]), treino[:T].numpy()) and np.array_equal(host(alvo[2]), treino[12346:12346 + T].numpy())
    reg.novo_passo(0)
    t2, a2 = tok[:2].contiguous(), alvo[:2].contiguous()
    with pytest.raises(ErroJatai) as e:
        c.janelas(torch.tensor([7, n - T]), T, t2, a2)
    msg = str(e.value)
    assert "janelas" in msg and f"valor    : {n - T}" in msg, msg
    assert reg.ultimo_evento.idx == 1 * T
    assert np.array_equal(host(t2[0]), treino[7:7 + T].numpy()) and np.array_equal(host(a2[0]), treino[8:8 + T].numpy())
    assert not host(t2[1]).any() and not host(a2[1]).any()
    reg.novo_passo(1)                           # a negative start is refused the same way
    with pytest.raises(ErroJatai) as e:
        c.janelas(torch.tensor([5, 9, -1]), T)
    assert "janelas" in str(e.value) and "valor    : -1" in str(e.value), str(e.value)
    assert reg.ultimo_evento.idx == 2 * T


def test_grafo_com_corpus_igual_ao_grafo_com_lotes(treino):
    """Two models from one seed (the reference shape, 2 layers): one graph fed the host batches of
    dados.lote, one that gathers the windows itself from the same generator state; 4 steps, then the same
    (d_alvo, soma) per step, weights, momenta and residuals. A start past the end inside the replayed graph then
    raises the sentinel naming janelas in scope "dados"."""
    from jatai_amd import dados as DD
    from jatai_amd.modelo import Modelo, PassoGravado
    from jatai_amd.registro import ErroJatai
    ops, reg = _ops(vigiar=False)
    f = TR.gold()["forma"]
    Bt, T = 8, f["T"]
    mk = lambda: Modelo(f["V"], f["D"], f["H"], f["FF"], 2, 3, "cuda", ops, reg)
    a, b = mk(), mk()
    c = DD.Corpus(ops, treino)
    ga, gb = torch.Generator().manual_seed(99), torch.Generator().manual_seed(99)
    tok, alvo = DD.lote(treino, ga, Bt, T, "cuda")
    reg.novo_passo(0); a.passo(tok, alvo, k_lr=4); reg.fim_passo()
    tb, ab = c.lote(gb, Bt, T)
    reg.novo_passo(0); b.passo(tb, ab, k_lr=4); reg.fim_passo()
    pa, pb = PassoGravado(a, Bt, T, 4), PassoGravado(b, Bt, T, 4, corpus=c)
    assert pb.lancamentos[0].op == "janelas" and len(pb.lancamentos) == len(pa.lancamentos) + 1
    with pytest.raises(RuntimeError):
        pb(tok, alvo)
    for p in range(1, 5):
        reg.novo_passo(p)
        x, y = DD.lote(treino, ga, Bt, T, "cuda")
        la = float(pa(x, y))
        lb = float(pb.de_corpus(gb))
        torch.cuda.synchronize()
        reg.fim_passo()
        assert la == lb and R.sha(host(pa.d_alvo)) == R.sha(host(pb.d_alvo)) and R.sha(host(pa.soma)) == R.sha(host(pb.soma)), p
    est = lambda m: [R.sha(host(t)) for n in m.p for t in (*m.p[n], *m.mom[n], *m.res[n])]
    assert est(a) == est(b)
    pb.ini.fill_(c.n - T)
    reg.novo_passo(5)
    with pytest.raises(ErroJatai) as e:
        reg.lancamentos = pb.lancamentos
        pb.grafo.replay()
        reg.fim_passo()
    assert "dados" in str(e.value) and "janelas" in str(e.value), str(e.value)
