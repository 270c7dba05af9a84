"""Writes long training-loss traces with the CPU oracle (oracle/libjatai_oracle.so through jatai_amd.modelo.Modelo
on OpsOraculo). Fixture writer only: it does not import the reference, and neither the tests nor the GPU box
run it.

  trace_r600.jsonl  the reference model shape of trace_r.json (V 256, D 256, 64 heads x 4, FF 1024, 12 layers,
                    Bt 8, T 128, BLK 128, k_lr 4): 600 steps. Before anything is written, the oracle's first
                    steps are checked against trace_r.json, which the reference spec wrote (modelo.py:51-140
                    with OpsRef), so the file extends the spec's own trace.
  trace_c4.jsonl    BASELINE config 4 (V 256, D 512, 8 heads x 64, FF 2048, 12 layers, Bt 8, T 256, BLK 32,
                    k_lr 4): as many steps as asked. Attention at head width 64 is the declared extension of the
                    spec (it reduces to the spec at head width 4), so this trace is anchored on the oracle alone.
  trace_c5.jsonl    BASELINE config 5 (the config-4 widths with 24 layers, Bt 64 x T 256 = 16384 tokens and the
                    16-bit residual stream, modelo.py:60-130): 10 steps (about 3-4 minutes each on 8 cores).

Both use seed-0 init (modelo.py:16-45) and the batches of tests/traco.py: uniform ids from substream 4242,
(x[:, :-1], x[:, 1:]) as treino_int8_gpu/treino.py:41-44. Line 1 holds the shape and the init hashes; each
further line one step: the SHA-256 of the integer softmax outputs d_alvo and soma (the loss is defined on
them) and the float64 loss mean(d/256 + ln(s/4096)) (modelo.py:93) as a hex float. Lines are appended and
flushed as steps finish into `<name>.parcial`, which replaces the fixture once every step is written.

Usage: python tests/golden/make_trace_oracle.py r600|c4|c5 [--passos N] [--threads T]
"""
import argparse
import json
import os
import sys
import time

import torch

AQUI = os.path.dirname(os.path.abspath(__file__))
RAIZ = os.path.dirname(os.path.dirname(AQUI))
sys.path.insert(0, RAIZ)
sys.path.insert(0, os.path.dirname(AQUI))
import recipe as R  # noqa: E402
import traco as TR  # noqa: E402

FORMAS = {
    "r600": dict(V=256, D=256, H=64, FF=1024, L=12, T=128, Bt=8, BLK=128, k_lr=4, semente=0, tokens_seed=4242),
    "c4": dict(V=256, D=512, H=8, FF=2048, L=12, T=256, Bt=8, BLK=32, k_lr=4, semente=0, tokens_seed=4242),
    "c5": dict(V=256, D=512, H=8, FF=2048, L=24, T=256, Bt=64, BLK=32, k_lr=4, semente=0, tokens_seed=4242, r16=True),
}
PASSOS = {"r600": 600, "c4": 600, "c5": 10}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("qual", choices=sorted(FORMAS))
    ap.add_argument("--passos", type=int, default=None)
    ap.add_argument("--threads", type=int, default=8)
    a = ap.parse_args()
    torch.set_num_threads(a.threads)
    os.environ.setdefault("OMP_NUM_THREADS", str(a.threads))
    from jatai_amd import ops as O
    from jatai_amd.modelo import Modelo, perda_de
    from oracle.ops_oracle import OpsOraculo
    f = FORMAS[a.qual]
    n = a.passos or PASSOS[a.qual]
    O.BLK = f["BLK"]
    m = Modelo(f["V"], f["D"], f["H"], f["FF"], f["L"], f["semente"], "cpu", OpsOraculo(f["BLK"]), TR.RegStub(),
               r16=f.get("r16", False))
    m.perda_inteira = True
    init = {k: [R.sha(t[0].numpy()), R.sha(t[1].numpy())] for k, t in m.p.items()}
    gold = TR.gold() if a.qual == "r600" else None
    if gold is not None:
        assert gold["forma"] == f and gold["init"] == init, "oracle model differs from the spec's trace"
    caminho = os.path.join(AQUI, f"trace_{a.qual}.jsonl")
    with open(caminho + ".parcial", "w") as out:
        out.write(json.dumps({"forma": f, "init": init}, separators=(",", ":")) + "\n")
        for p in range(n):
            t0 = time.time()
            tok, alvo = TR.lote(p, f["Bt"], f["T"], f["V"], "cpu")
            d, s = m.passo(tok, alvo, k_lr=f["k_lr"])
            perda = float(perda_de(d, s))
            ent = {"passo": p, "d_alvo": R.sha(d.numpy()), "soma": R.sha(s.numpy()), "perda_hex": perda.hex()}
            if gold is not None and p < len(gold["passos"]):
                g = gold["passos"][p]
                assert (ent["d_alvo"], ent["soma"]) == (g["d_alvo"], g["soma"]), f"step {p} differs from the spec"
                assert perda == g["perda"], f"step {p}: loss {perda!r} vs spec {g['perda']!r}"
            out.write(json.dumps(ent, separators=(",", ":")) + "\n")
            out.flush()
            print(f"{a.qual} passo {p}: loss {perda:.6f}  {time.time() - t0:.1f}s", flush=True)
    os.replace(caminho + ".parcial", caminho)
    O.BLK = 128


if __name__ == "__main__":
    main()
