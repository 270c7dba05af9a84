"""Runs the training step at the reference model shape and records every op output, for comparison with the
traces written from the reference spec (Modelo.passo with OpsRef, modelo.py:51-140): tests/golden/trace_r.json
(Bt = 8, the reference's `conferir` batch) and tests/golden/trace_r_bt16.json (Bt = 16, the batch of its speed
runs)."""
import contextlib
import json
import os

import torch

import cases as CS
import recipe as R

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TRACOS = ("trace_r.json", "trace_r_bt16.json")


def gold(nome="trace_r.json"):
    return json.load(open(os.path.join(GOLDEN, nome)))


class RegStub:
    @contextlib.contextmanager
    def trecho(self, nome):
        yield

    def info(self, *a, **k):
        pass


def lote(p, Bt, T, V, dev):
    """Step p's batch: uniform ids, (x[:, :-1], x[:, 1:]) as in treino_int8_gpu/treino.py:41-44."""
    x = R.tokens(R.substream(4242, f"passo {p}"), Bt * (T + 1), V).reshape(Bt, T + 1)
    tok = torch.from_numpy(x[:, :-1].copy()).long().to(dev)
    alvo = torch.from_numpy(x[:, 1:].copy()).long().to(dev)
    return tok, alvo


def roda(ops, reg, dev, passos, host, nome="trace_r.json"):
    """Builds the model exactly as the golden writer did and runs `passos` steps; returns (init hashes, steps)."""
    from jatai_amd.modelo import Modelo
    g = gold(nome)
    f = g["forma"]
    rec = CS.Gravador(ops, host)
    m = Modelo(f["V"], f["D"], f["H"], f["FF"], f["L"], f["semente"], dev, rec, reg)
    m.otimizador_fundido = False        # the trace records momento, peso and transpoe per tensor, in the spec's order
    m.transpostas_em_lote = False
    m.dw_em_lote = False
    m.quant_na_atencao = False
    m.transposta_na_gemm = False
    m.transposta_na_relu2 = False
    m.rms_soma = False
    m.soma16_fundida = False
    m.perda_fundida = False
    init = {n: [R.sha(host(t[0])), R.sha(host(t[1]))] for n, t in m.p.items()}
    out = []
    for p in range(passos):
        rec.log = []
        tok, alvo = lote(p, f["Bt"], f["T"], f["V"], dev)
        perda = float(m.passo(tok, alvo, k_lr=f["k_lr"]))
        out.append({"perda": perda, "chamadas": [[op, list(h)] for op, h in rec.log]})
    return m, init, out


def confere(init, passos, nome="trace_r.json"):
    """Asserts init hashes and every op output of each step against the golden trace."""
    g = gold(nome)
    assert init == g["init"], "initial weights differ from the reference init (modelo.py:16-45)"
    for p, ent in enumerate(passos):
        gp = g["passos"][p]
        esperado = [[op, list(h)] for op, h in gp["chamadas"]]
        assert len(ent["chamadas"]) == len(esperado) == 522
        for k, (a, b) in enumerate(zip(ent["chamadas"], esperado)):
            assert a == b, f"step {p}, op #{k} '{b[0]}': outputs differ from the spec"
        assert abs(ent["perda"] - gp["perda"]) <= 1e-12 * abs(gp["perda"]), (ent["perda"], gp["perda"])
