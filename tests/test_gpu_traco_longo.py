"""Long loss traces: the fused training step, captured once as a hipGraph and replayed, reproduces step after step
the integer softmax outputs (d_alvo, soma) of the CPU oracle's trace, hence the float64 loss bit for bit
(mean(d/256 + ln(s/4096)), modelo.py:93, evaluated on the host from the GPU's integers).

  trace_r600.jsonl  600 steps at the reference model shape (BLK 128, 64 heads x 4); its first 32 steps are the
                    reference spec's own (trace_r.json), the rest the oracle's extension of them;
  trace_c4.jsonl    BASELINE config 4 (D 512, 8 heads x 64, FF 2048, 12 layers, Bt 8, T 256, BLK 32): the
                    steps the oracle wrote, from ops pinned by the reference's goldens and an attention extension
                    pinned by the head-width-4 reductions, the v = 0 closed form and the head-dimension
                    permutation tests (tests/test_oracle.py);
  trace_c5.jsonl    BASELINE config 5 at its workload: 24 layers, Bt 64 x T 256 = 16384 tokens, the 16-bit
                    residual stream (modelo.py:60-130) -- the step bench.py times, with its grouped
                    weight-gradient GEMMs at K = 16384: 10 steps.

Both fixtures come from tests/golden/make_trace_oracle.py."""
import json
import os

import pytest
import torch

import recipe as R
import traco as TR
from backends import LOGS, host

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _le(nome):
    caminho = os.path.join(GOLD, nome)
    if not os.path.exists(caminho):
        pytest.skip(f"{nome} not written")
    linhas = [json.loads(x) for x in open(caminho) if x.strip()]
    return linhas[0], linhas[1:]


@pytest.mark.parametrize("nome", ["trace_r600.jsonl", "trace_c4.jsonl", "trace_c5.jsonl"])
def test_traco_longo_grafo(nome):
    from jatai_amd import ops as O
    from jatai_amd.modelo import Modelo, PassoGravado, perda_de
    from jatai_amd.registro import Registro
    cab, passos = _le(nome)
    f = cab["forma"]
    assert len(passos) >= 2
    O.BLK = f["BLK"]
    try:
        reg = Registro(LOGS, "traco_longo", eco=False)
        m = Modelo(f["V"], f["D"], f["H"], f["FF"], f["L"], f["semente"], "cuda", O.OpsHip(reg), reg, r16=f.get("r16", False))
        assert {n: [R.sha(host(t[0])), R.sha(host(t[1]))] for n, t in m.p.items()} == cab["init"]
        pg = PassoGravado(m, f["Bt"], f["T"], f["k_lr"])
        print(f"{nome}: {len(passos)} steps, {len(pg.lancamentos)} launches per replay", flush=True)
        for ent in passos:
            p = ent["passo"]
            tok, alvo = TR.lote(p, f["Bt"], f["T"], f["V"], "cuda")
            reg.novo_passo(p)
            pg(tok, alvo)
            torch.cuda.synchronize()
            reg.fim_passo()
            d, s = host(pg.d_alvo), host(pg.soma)
            assert (R.sha(d), R.sha(s)) == (ent["d_alvo"], ent["soma"]), f"{nome}: step {p} differs from the oracle"
            perda = float(perda_de(torch.from_numpy(d), torch.from_numpy(s)))
            assert perda.hex() == ent["perda_hex"], f"{nome}: step {p} loss {perda!r}"
    finally:
        O.BLK = 128
