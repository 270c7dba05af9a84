"""The byte-level data path of the reference's training drivers (treino_int8_gpu/treino.py:29-44, which the CUDA
driver imports as its data module, jatai_cuda/treino_cuda.py:22,38-45; jatai_cuda/noite.py:35-43 reads whole files).

The corpus is two JSONL files, `Portuguese.jsonl` then `English.jsonl`, one `{"text": ...}` object per line. Each
line's text, UTF-8 encoded and followed by b"\\n\\n", goes to the validation bytes when its line index within its
file is a multiple of 20 and to the training bytes otherwise. `carregar` reads the first 3000 lines of each file
(treino.py:29-38), `carregar_tudo` every line (noite.py:35-43). Tokens are the bytes themselves (V = 256).

`lote` draws a batch with the same generator calls as treino.py:41-44, so one generator state gives the
reference's batch: Bt window starts from `torch.randint(0, n - T - 1, (Bt,), generator=g)` (a start is at most
n - T - 2), windows of T + 1 bytes, inputs the first T and targets the last T.

`Corpus` keeps the training bytes in device memory (HBM holds any corpus of this kind whole) and writes a batch's
windows straight into int32 token buffers with one kernel (`OpsHip.janelas`, `jt_janelas`): the host sends the Bt
int64 starts, 8 bytes per sequence, instead of 2 x Bt x T int64 tokens, and no int64 -> int32 conversion runs.
`jatai_amd.modelo.PassoGravado` takes a `Corpus` and captures that kernel as the graph's first node.
"""
import json
import os

import numpy as np
import torch

LINGUAS = ("Portuguese", "English")
LINHAS = 3000          # lines read per language by carregar (treino.py:34)
VAL_CADA = 20          # every 20th line of a file (index 0, 20, 40, ...) is validation (treino.py:37)
SEPARADOR = b"\n\n"    # appended to each line's text (treino.py:36)


def pasta_padrao():
    """The corpus folder: $JATAI_DADOS, as in treino.py:22."""
    p = os.environ.get("JATAI_DADOS")
    if not p:
        raise FileNotFoundError("no corpus folder: set JATAI_DADOS to the folder holding Portuguese.jsonl and English.jsonl")
    return p


def _bytes_long(b):
    """bytes -> int64 tensor of the byte values (torch.tensor(list(b), dtype=torch.long) without the list)."""
    return torch.from_numpy(np.frombuffer(bytes(b), dtype=np.uint8).astype(np.int64))


def divide(pasta=None, linhas=LINHAS):
    """(training bytes, validation bytes) of the corpus in `pasta`, `linhas` lines per language (None: all)."""
    pasta = pasta or pasta_padrao()
    partes = {True: bytearray(), False: bytearray()}           # True: validation
    for lingua in LINGUAS:
        with open(os.path.join(pasta, f"{lingua}.jsonl"), encoding="utf-8") as f:
            for i, linha in enumerate(f):
                if linhas is not None and i >= linhas:
                    break
                partes[i % VAL_CADA == 0] += json.loads(linha)["text"].encode("utf-8") + SEPARADOR
    return bytes(partes[False]), bytes(partes[True])


def carregar(pasta=None, linhas=LINHAS):
    """treino.py:29-38: (training, validation) as int64 tensors of byte values."""
    treino, val = divide(pasta, linhas)
    return _bytes_long(treino), _bytes_long(val)


def carregar_tudo(pasta=None):
    """noite.py:35-43: every line of both files."""
    return carregar(pasta, None)


def inicios(n, gerador, Bt, T):
    """The Bt window starts of one batch over n bytes, drawn as treino.py:42 draws them."""
    if n < T + 2:
        raise ValueError(f"corpus of {n} bytes is too short for windows of {T + 1}")
    return torch.randint(0, n - T - 1, (Bt,), generator=gerador)


def lote(dados, gerador, Bt, T, dev="cpu"):
    """treino.py:41-44: (inputs, targets), each [Bt, T] int64 on `dev`, views of one [Bt, T + 1] window tensor."""
    ini = inicios(len(dados), gerador, Bt, T)
    x = dados[ini[:, None] + torch.arange(T + 1)].to(dev)
    return x[:, :-1], x[:, 1:]


class Corpus:
    """Training bytes resident in device memory; `lote` writes a batch's windows into int32 buffers on the device
    with the same starts as `lote(dados, gerador, Bt, T)` for the same generator state."""

    def __init__(self, ops, dados, dev="cuda"):
        if dados.dtype != torch.uint8 and (int(dados.min()) < 0 or int(dados.max()) > 255):
            raise ValueError("corpus values must be bytes (0..255)")
        self.ops, self.dev = ops, torch.device(dev)
        self.bytes = dados.to(torch.uint8).to(self.dev).contiguous()
        self.n = self.bytes.numel()

    def inicios(self, gerador, Bt, T):
        return inicios(self.n, gerador, Bt, T)

    def janelas(self, ini, T, tok=None, alvo=None):
        """Windows from given starts (int64, host or device) into tok / alvo (int32 [Bt, T], made if None)."""
        ini = ini.to(self.dev, torch.int64)
        return self.ops.janelas(self.bytes, ini, T, tok, alvo)

    def lote(self, gerador, Bt, T, tok=None, alvo=None):
        return self.janelas(self.inicios(gerador, Bt, T), T, tok, alvo)
