"""Writes dados.json: the reference's byte data path run on the synthetic corpus of tests/recipe.py.

Run ONLY in a container that holds the reference checkout (default /root/reference); never on the GPU box and never
by the tests. It writes the synthetic corpus (`recipe.corpus_sintetico`) into a temporary folder, points the
reference's data module at it (`treino_int8_gpu/treino.py`, module constants DADOS, T, BT, DEV) and stores only data:
the SHA-256, length and leading bytes of the training and validation bytes of `carregar` (treino.py:29-38), and for
each (seed, Bt, T) the window starts and the SHA-256 of the inputs and targets of `lote` (treino.py:41-44) drawn with
`torch.Generator().manual_seed(seed)`, three batches in a row from one generator.

Usage: python tests/golden/make_dados.py [--ref /root/reference]
"""
import argparse
import hashlib
import json
import os
import sys
import tempfile

import numpy as np
import torch

AQUI = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(AQUI))
import recipe as R  # noqa: E402

CASOS = ((7, 8, 128), (123, 8, 128), (5, 16, 128), (11, 3, 5), (13, 4, 256))


def sha(t):
    return hashlib.sha256(np.ascontiguousarray(t.cpu().numpy().astype(np.int64)).tobytes()).hexdigest()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    a = ap.parse_args()
    pasta = tempfile.mkdtemp()
    R.corpus_sintetico(pasta)
    sys.path.insert(0, os.path.join(a.ref, "treino_int8_gpu"))
    import treino  # noqa: E402  (the reference's data module)
    treino.DADOS, treino.DEV = pasta, "cpu"
    tr, val = treino.carregar()
    out = dict(corpus=dict(semente=1),
               carregar=dict(treino=dict(n=len(tr), sha=sha(tr), inicio=tr[:64].tolist()),
                             val=dict(n=len(val), sha=sha(val), inicio=val[:64].tolist())),
               lotes=[])
    for semente, Bt, T in CASOS:
        treino.BT, treino.T = Bt, T
        g = torch.Generator().manual_seed(semente)
        passos = []
        for _ in range(3):
            estado = g.get_state()
            x, y = treino.lote(tr, g)
            g2 = torch.Generator()
            g2.set_state(estado)
            ini = torch.randint(0, len(tr) - T - 1, (Bt,), generator=g2)   # the starts lote drew, for the record
            assert torch.equal(x[:, 0], tr[ini]), "starts of the recorded windows"
            passos.append(dict(ini=ini.tolist(), x=sha(x), y=sha(y), x0=x[0, :16].tolist()))
        out["lotes"].append(dict(semente=semente, Bt=Bt, T=T, passos=passos))
    with open(os.path.join(AQUI, "dados.json"), "w") as f:
        json.dump(out, f, indent=1)
    print("dados.json:", len(tr), "training bytes,", len(val), "validation bytes,", len(CASOS), "batch cases")


if __name__ == "__main__":
    main()
