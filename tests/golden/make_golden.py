"""Writes the golden fixtures of this directory from the reference's executable int64 specification.

Run ONLY in a container that holds the reference checkout (default /root/reference); never on the GPU box and
never by the tests. It imports `jatai_cuda/ops.py` (class `OpsRef`, the spec, ops.py:92-290) and
`jatai_cuda/modelo.py` (the step composition, modelo.py:16-140) on the CPU, runs them on inputs from
`tests/recipe.py`, and stores only data: per-output SHA-256 hashes, shapes and a few leading values.

Fixtures:
  ops_blk128.json   the 40 op cases of tests/cases.py (teste_ops.py:57-98) with the spec at BLK=128
  ops_blk32.json    the same cases with the spec's block constant set to 32 (ops.BLK is a module global the
                    spec reads everywhere: quant, expande, gemm, g_rms, _alinha)
  ops_dominio_blk128.json, ops_dominio_blk32.json
                    the cases of tests/cases.py casos_dominio(): the rest of the reference's shape domain (row
                    widths that are not powers of two, attention at H = 32 and T = 32, 96)
  config1.json      BASELINE config 1: one 512x512x512 GEMM, exponents uniform in [-8, 0], at BLK 32 and 128
  primitives.json   exp_int over its whole domain, isqrt / bitlen / rnd on sampled inputs
  trace_r.json      every op output of two full training steps (Modelo.passo with k_lr=4) at the reference
                    model shape (V=256, D=256, H=64, FF=1024, L=12, T=128, Bt=8), plus the per-step
                    (d_alvo, soma) hashes and float64 losses of N further steps
  trace_r_bt16.json the same at Bt=16 (2048 tokens per step: the batch of the reference's own speed runs,
                    treino_cuda.py:119-165, bench_grafo.py:29-37)

Usage: python tests/golden/make_golden.py [--ref /root/reference] [--only ops|dominio|config1|prim|trace|trace16]
       [--passos N]
"""
import argparse
import contextlib
import json
import math
import os
import sys
import time

import numpy as np
import torch

AQUI = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(AQUI))
import cases as CS  # noqa: E402
import recipe as R  # noqa: E402


def host(t):
    return t.detach().cpu().numpy()


def set_blk(O, blk):
    """The spec reads the block size from the module global ops.BLK, except `expande(E, b=BLK)`, whose default
    was bound when ops.py was imported (ops.py:54); both are set so every function of the spec uses `blk`."""
    O.BLK = blk
    O.expande.__defaults__ = (blk,)


class Backend:
    def __init__(self, O):
        self.O = O
        self.ops = O.OpsRef()

    def dev(self, a):
        return torch.from_numpy(np.ascontiguousarray(a))

    def limite(self, flag):
        old = self.O.ATENCAO_LIMITE
        self.O.ATENCAO_LIMITE = flag
        return old


def run_ops(O, blk, casos=None):
    set_blk(O, blk)
    be = Backend(O)
    out = []
    for i, (nome, fn) in enumerate(casos or CS.casos()):
        t0 = time.time()
        rec = CS.Gravador(be.ops, host)
        g = CS.Gen(R.substream(1000 + i, nome), blk, be.dev)
        res = fn(rec, g, be)
        heads = [host(t).reshape(-1)[:8].tolist() for t in CS.plano(res)]
        out.append({"nome": nome, "seed": 1000 + i, "chamadas": rec.log, "inicio": heads})
        print(f"  blk {blk} {nome}: {time.time() - t0:.1f}s", flush=True)
    set_blk(O, 128)
    return out


def run_config1(O):
    out = {}
    for blk in (32, 128):
        set_blk(O, blk)
        ops = O.OpsRef()
        a = R.bloco(R.substream(0, "A"), 512, 512, blk, espalha=4, e0=-4)
        b = R.bloco(R.substream(0, "B"), 512, 512, blk, espalha=4, e0=-4)
        A = tuple(torch.from_numpy(x) for x in a)
        B = tuple(torch.from_numpy(x) for x in b)
        C = ops.gemm(A, B)
        Cc = ops.gemm(A, B, cru=True)
        out[str(blk)] = {"bloco": [R.sha(host(t)) for t in C], "cru": [R.sha(host(t)) for t in Cc],
                         "inicio": host(C[0]).reshape(-1)[:16].tolist(), "E": host(C[1]).reshape(-1)[:16].tolist()}
    set_blk(O, 128)
    return out


def run_prim(O):
    d = torch.arange(0, 7001, dtype=torch.int64)
    ex = O.exp_int(d)
    n = torch.from_numpy(np.concatenate([np.arange(0, 70000), R.uniform_int(7, (200000,), 0, (1 << 30) - 1)]).astype(np.int64))
    iq = O.isqrt(n)
    x = torch.from_numpy(R.uniform_int(8, (100000,), -(1 << 29), (1 << 29) - 1))
    s = torch.from_numpy(R.uniform_int(9, (100000,), -8, 40))
    rn = O.rnd(x, s)
    bl = O.bitlen(x)
    return {"exp_int": {"n": 7001, "sha": R.sha(host(ex)), "inicio": host(ex)[:16].tolist()},
            "isqrt": {"sha": R.sha(host(iq))},
            "rnd": {"x_seed": 8, "s_seed": 9, "n": 100000, "sha": R.sha(host(rn))},
            "bitlen": {"sha": R.sha(host(bl))}}


class RegStub:
    @contextlib.contextmanager
    def trecho(self, nome):
        yield

    def info(self, *a, **k):
        pass


def run_trace(O, MO, passos_extra, Bt=8, blk=128):
    set_blk(O, blk)
    V, D, H, FF, L, T = 256, 256, 64, 1024, 12, 128
    rec = CS.Gravador(O.OpsRef(), host)
    m = MO.Modelo(V, D, H, FF, L, 0, "cpu", rec, RegStub())
    init = {n: [R.sha(host(t[0])), R.sha(host(t[1]))] for n, t in m.p.items()}
    passos = []
    for p in range(2 + passos_extra):
        x = R.tokens(R.substream(4242, f"passo {p}"), Bt * (T + 1), V).reshape(Bt, T + 1)
        tok, alvo = torch.from_numpy(x[:, :-1].copy()).long(), torch.from_numpy(x[:, 1:].copy()).long()
        rec.log = []
        t0 = time.time()
        perda = float(m.passo(tok, alvo, k_lr=4))
        sm = [c for c in rec.log if c[0] == "softmax_ce"][0]
        ent = {"passo": p, "perda": perda, "perda_hex": perda.hex(), "d_alvo": sm[1][2], "soma": sm[1][3],
               "n_ops": len(rec.log)}
        if p < 2:
            ent["chamadas"] = rec.log
        passos.append(ent)
        print(f"  passo {p}: loss {perda:.6f}  {len(rec.log)} ops  {time.time() - t0:.1f}s", flush=True)
    set_blk(O, 128)
    return {"forma": dict(V=V, D=D, H=H, FF=FF, L=L, T=T, Bt=Bt, BLK=blk, k_lr=4, semente=0, tokens_seed=4242),
            "init": init, "passos": passos}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    ap.add_argument("--only", default="all")
    ap.add_argument("--passos", type=int, default=0)
    ap.add_argument("--threads", type=int, default=8)
    a = ap.parse_args()
    torch.set_num_threads(a.threads)
    sys.path.insert(0, os.path.join(a.ref, "jatai_cuda"))
    import ops as O       # noqa: E402  the reference spec (CPU only; OpsCuda is never instantiated)
    import modelo as MO   # noqa: E402
    w = lambda nome, obj: json.dump(obj, open(os.path.join(AQUI, nome), "w"), separators=(",", ":"))
    if a.only in ("all", "prim"):
        w("primitives.json", run_prim(O))
    if a.only in ("all", "config1"):
        w("config1.json", run_config1(O))
    if a.only in ("all", "ops"):
        for blk in (128, 32):
            w(f"ops_blk{blk}.json", run_ops(O, blk))
    if a.only in ("all", "dominio"):
        for blk in (128, 32):
            w(f"ops_dominio_blk{blk}.json", run_ops(O, blk, CS.casos_dominio()))
    if a.only in ("all", "trace"):
        w("trace_r.json", run_trace(O, MO, a.passos))
    if a.only in ("all", "trace16"):
        w("trace_r_bt16.json", run_trace(O, MO, a.passos, Bt=16))


if __name__ == "__main__":
    main()
