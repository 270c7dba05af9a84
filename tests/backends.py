"""Backends with the reference operator surface, for the parity tests: the GPU path (OpsHip, through the C ABI
of libjatai.so) and the CPU oracle (tests only)."""
import os
import tempfile

import numpy as np
import torch

import recipe as R

LOGS = os.path.join(tempfile.gettempdir(), "jatai_testes")


def host(t):
    return t.detach().cpu().numpy()


class GPU:
    def __init__(self, blk, vigiar=False):
        from jatai_amd import ops as O
        from jatai_amd.registro import Registro
        self.O = O
        O.BLK = blk
        self.reg = Registro(LOGS, "testes", vigiar=vigiar, eco=False)
        self.ops = O.OpsHip(self.reg)
        self.reg.novo_passo(0)

    def dev(self, a):
        return torch.from_numpy(np.ascontiguousarray(a)).cuda()

    def limite(self, flag):
        old, self.O.ATENCAO_LIMITE = self.O.ATENCAO_LIMITE, flag
        return old


class CPU:
    def __init__(self, blk):
        from oracle.ops_oracle import OpsOraculo
        self.ops = OpsOraculo(blk)

    def dev(self, a):
        return torch.from_numpy(np.ascontiguousarray(a))

    def limite(self, flag):
        old, self.ops.limite = self.ops.limite, flag
        return old


def primeira_diferenca(a, b):
    """(flat index, a value, b value, count) of the first difference of two arrays, or None."""
    a, b = np.asarray(a).reshape(-1), np.asarray(b).reshape(-1)
    if a.shape != b.shape:
        return ("forma", a.shape, b.shape, -1)
    d = np.nonzero(a != b)[0]
    if d.size == 0:
        return None
    i = int(d[0])
    return (i, a[i].item(), b[i].item(), int(d.size))


def sha_lista(ts):
    return [R.sha(host(t)) for t in ts]
