"""Throughput of the INT8 integer training step on one MI355X, with the roofline of its dominant kernel and the CPU
oracle timed on the same host as the baseline.

A step is one hipGraph replay of the whole training step (forward, backward, momentum + error-feedback update of
every weight) over one synthetic batch of uniform random token ids, following the reference's tokens/s protocol
(jatai_cuda/treino_cuda.py:119-151): copy the batch into the graph's input buffers, clear the device error record,
replay, read the error record. Batches are resident in HBM before the timed region.

Workloads (--config):
  b4  BASELINE config 4 (default): 12 layers, D=512, 8 heads x 64, FF=2048, V=256, T=256, Bt=8 (2048 tokens),
      BLK=32
  r   reference-native shape: 12 layers, D=256, 64 heads x 4, FF=1024, T=128, Bt=16 (2048 tokens), BLK=128 --
      the configuration of the reference's published 34,248 tokens/s (GTX 1650, README.md:87)

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config b4|r] [--no-cpu]
Prints one JSON line.
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "INT8 train tokens/s (12L, 2048 tok); block-32 GEMM TOPS & % i8 MFMA peak"
PEAK_I8 = 5.0e15          # MI355X dense int8 MFMA, ops/s
PEAK_HBM = 8.0e12         # bytes/s

CONFIGS = {
    "b4": dict(V=256, D=512, H=8, FF=2048, L=12, T=256, Bt=8, BLK=32, r16=False,
               nome="BASELINE config 4: 12L D512 H8x64 FF2048 V256 T256 Bt8 BLK32", publicado=None),
    "r": dict(V=256, D=256, H=64, FF=1024, L=12, T=128, Bt=16, BLK=128, r16=False,
              nome="reference-native 12L D256 H64x4 FF1024 T128 Bt16 BLK128", publicado=34248.0),
}


def args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="b4", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--so-passo", action="store_true", help="time the step only (no GEMM sweep, no CPU baseline): for profiling")
    ap.add_argument("--trafego", action="store_true",
                    help="for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE: a 256 MiB device copy (the counters' calibration), "
                         "then each GEMM shape of the step twice in its mode; prints the dispatch order")
    return ap.parse_args()


def gemm_formas(c):
    """(M, N, K, mode, count) of every GEMM of one step (modelo.py:51-134), one entry per distinct shape and mode:
    mode 0 block output, 1 raw, 2 + residual add, 3 + ReLU^2, 4 ReLU^2 backward."""
    M, D, FF, V, L = c["Bt"] * c["T"], c["D"], c["FF"], c["V"], c["L"]
    f = {}

    def add(n, m, nn, k, modo, cont):
        f[n] = (m, nn, k, modo, f.get(n, (0, 0, 0, 0, 0))[4] + cont)
    add("fwd qkv", M, 3 * D, D, 0, L)
    add("fwd out-proj+soma", M, D, D, 2, L)
    add("fwd ffn-up+relu2", M, FF, D, 3, L)
    add("fwd ffn-down+soma", M, D, FF, 2, L)
    add("logits", M, V, D, 1, 1)
    add("dX out", M, D, V, 0, 1)
    add("dX ffn-down+relu2_back", M, FF, D, 4, L)
    add("dX ffn-up", M, D, FF, 0, L)
    add("dX out-proj", M, D, D, 0, L)
    add("dX qkv", M, D, 3 * D, 0, L)
    add("dW qkv", 3 * D, D, M, 1, L)
    add("dW out-proj", D, D, M, 1, L)
    add("dW ffn-up", FF, D, M, 1, L)
    add("dW ffn-down", D, FF, M, 1, L)
    add("dW out", V, D, M, 1, 1)
    add("dW emb", V, D, M, 1, 1)
    return f


def gemm_kernel(O, ops, M, N, K, modo):
    """Symbol and grid the library launches for this shape, to match rocprof rows."""
    ks = ops.lib.jt_gemm_divisoes(M, N, K, modo)
    return {"symbol": f"k_gemm<{O.BLK}, {modo}, {ks}>", "workgroups": (M // 32) * (N // 128), "threads": 256 * ks}


def mede_gemms(O, ops, c, rep=20):
    """Average launch duration of each GEMM shape: `rep` launches of one shape captured as one hipGraph (on the
    stream the library launches on, so launch gaps are the graph's, as in the training step), timed with HIP
    events on that stream around the replay; inputs resident in HBM; 2MNK / duration."""
    import torch
    blk = c["BLK"]
    out = {}
    g = torch.Generator().manual_seed(3)

    def bloco(R, C, e0):
        m = torch.randint(-127, 128, (R, C), generator=g, dtype=torch.int8).cuda()
        E = (e0 + torch.randint(-3, 4, (R, C // blk), generator=g)).to(torch.int8).cuda()
        return m, E
    for nome, (M, N, K, modo, cont) in gemm_formas(c).items():
        A, B, X = bloco(M, K, -8), bloco(N, K, -12), bloco(M, N, -6)
        saida = ops.gemm(A, B, cru=True) if modo == 1 else None
        chama = {0: lambda: ops.gemm(A, B), 1: lambda: ops.gemm(A, B, cru=True, saida=saida), 2: lambda: ops.gemm_soma(A, B, X),
                 3: lambda: ops.gemm_relu2(A, B), 4: lambda: ops.gemm_relu2_back(A, B, X)}[modo]
        chama()
        torch.cuda.synchronize()
        grafo = torch.cuda.CUDAGraph()
        with torch.cuda.graph(grafo):
            ops.lib.jt_stream(torch.cuda.current_stream().cuda_stream)
            try:
                for _ in range(rep):
                    chama()
            finally:
                ops.lib.jt_stream(None)
        grafo.replay()
        torch.cuda.synchronize()
        s = torch.cuda.Stream()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        with torch.cuda.stream(s):
            ev[0].record(s)
            for _ in range(3):
                grafo.replay()
            ev[1].record(s)
        torch.cuda.synchronize()
        ms = ev[0].elapsed_time(ev[1]) / (3 * rep)
        out[nome] = dict(M=M, N=N, K=K, modo=modo, por_passo=cont, ms=ms, tops=2 * M * N * K / (ms * 1e-3) / 1e12,
                         kernel=gemm_kernel(O, ops, M, N, K, modo))
        del grafo
    return out


def trafego_despacha(O, ops, c):
    """Dispatches for the HBM-traffic counter runs: one plain copy of 256 MiB, then every GEMM shape twice (the
    second launch of each is the one summarized), printed in launch order."""
    import torch
    x = torch.ones(256 << 20, dtype=torch.int8, device="cuda")
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    y.copy_(x)
    torch.cuda.synchronize()
    print("dispatch: copy 268435456 bytes", flush=True)
    del x, y
    blk = c["BLK"]
    g = torch.Generator().manual_seed(3)

    def bloco(R, C, e0):
        m = torch.randint(-127, 128, (R, C), generator=g, dtype=torch.int8).cuda()
        E = (e0 + torch.randint(-3, 4, (R, C // blk), generator=g)).to(torch.int8).cuda()
        return m, E
    for nome, (M, N, K, modo, cont) in gemm_formas(c).items():
        A, B, X = bloco(M, K, -8), bloco(N, K, -12), bloco(M, N, -6)
        chama = {0: lambda: ops.gemm(A, B), 1: lambda: ops.gemm(A, B, cru=True), 2: lambda: ops.gemm_soma(A, B, X),
                 3: lambda: ops.gemm_relu2(A, B), 4: lambda: ops.gemm_relu2_back(A, B, X)}[modo]
        torch.cuda.synchronize()
        for _ in range(2):
            chama()
            torch.cuda.synchronize()
        print(f"dispatch: {nome} {gemm_kernel(O, ops, M, N, K, modo)['symbol']} x2", flush=True)


def trafego(nome):
    """HBM bytes per launch of a GEMM shape from the committed counter summary (rocprofv3 --pmc FETCH_SIZE and
    WRITE_SIZE, each scaled by the same counter on a plain copy of known size), or None if it has no line for it."""
    arq = os.path.join(ROOT, "profiles", "gemm_hbm_traffic.txt")
    if not os.path.exists(arq):
        return None
    for linha in open(arq):
        if linha.startswith(nome + ":") and "traffic_bytes=" in linha:
            return int(linha.split("traffic_bytes=")[1].split()[0])
    return None


def cpu_baseline(c, segundos):
    """The CPU oracle (int64 C++ restatement of the spec, OpenMP) running the same model's training step on a
    bounded sample: batches of 2 sequences until `segundos` of wall time, tokens/s = tokens / wall."""
    import torch
    from jatai_amd import ops as O
    from jatai_amd.modelo import Modelo
    from oracle.ops_oracle import OpsOraculo

    class Nada:
        def trecho(self, n):
            import contextlib
            return contextlib.nullcontext()
    O.BLK = c["BLK"]
    m = Modelo(c["V"], c["D"], c["H"], c["FF"], c["L"], 0, "cpu", OpsOraculo(c["BLK"]), Nada(), r16=c["r16"])
    g = torch.Generator().manual_seed(11)
    bt = 2
    n = 0
    t0 = time.perf_counter()
    while True:
        x = torch.randint(0, c["V"], (bt, c["T"] + 1), generator=g)
        m.passo(x[:, :-1], x[:, 1:], k_lr=4)
        n += 1
        dt = time.perf_counter() - t0
        if dt >= segundos:
            break
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return dict(value=n * bt * c["T"] / dt, unit="tokens/s", cores=threads, kind="port",
                sample=f"{n} training steps of the same {c['L']}-layer model at Bt={bt} x T={c['T']} on the int64 CPU oracle "
                       f"(oracle/jatai_oracle.cpp, OpenMP {threads} threads), {dt:.1f} s")


def main():
    a = args()
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {a.gpus}); the multi-GPU path is a design "
              f"(DESIGN.md), not a measured configuration.", file=sys.stderr)
        sys.exit(2)
    import torch
    from jatai_amd import ops as O
    from jatai_amd.modelo import Modelo, PassoGravado
    from jatai_amd.registro import Registro

    c = CONFIGS[a.config]
    O.BLK = c["BLK"]
    reg = Registro("/tmp/jatai_bench", "bench", eco=False)
    ops = O.OpsHip(reg)
    if a.trafego:
        trafego_despacha(O, ops, c)
        return
    dev = "cuda"
    m = Modelo(c["V"], c["D"], c["H"], c["FF"], c["L"], 0, dev, ops, reg, r16=c["r16"])
    g = torch.Generator().manual_seed(1)
    nlotes = 6
    lotes = []
    for _ in range(nlotes):
        x = torch.randint(0, c["V"], (c["Bt"], c["T"] + 1), generator=g).to(dev)
        lotes.append((x[:, :-1].contiguous(), x[:, 1:].contiguous()))
    reg.novo_passo(0)
    m.passo(*lotes[0], k_lr=4)
    reg.fim_passo()
    pg = PassoGravado(m, c["Bt"], c["T"], 4)
    nlanc = len(pg.lancamentos)

    def passo(i):
        reg.novo_passo(i)
        perda = pg(*lotes[i % nlotes])
        reg.fim_passo()
        return perda
    for i in range(a.warmup):
        passo(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(a.steps):
        perda = passo(i)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    perda = float(perda)
    tokens = c["Bt"] * c["T"]
    tps = tokens * a.steps / dt

    if a.so_passo:
        print(json.dumps({"metric": METRIC, "value": tps, "unit": "tokens/s", "ms_per_step": dt / a.steps * 1e3,
                          "steps": a.steps, "warmup": a.warmup, "graph_launches": nlanc, "config": c["nome"]}), flush=True)
        return
    gem = mede_gemms(O, ops, c)
    tot_gemm_ms = sum(v["ms"] * v["por_passo"] for v in gem.values())
    dom_nome, dom = max(gem.items(), key=lambda kv: kv[1]["ms"] * kv[1]["por_passo"])
    achieved = 2 * dom["M"] * dom["N"] * dom["K"] / (dom["ms"] * 1e-3)
    roof = {"bound": "mfma", "achieved": achieved / 1e12, "peak": PEAK_I8 / 1e12, "unit": "TOP/s",
            "frac": achieved / PEAK_I8, "traffic": trafego(dom_nome),
            "kernel": f"{dom['kernel']['symbol']} ({dom_nome} M={dom['M']} N={dom['N']} K={dom['K']}, "
                      f"{dom['kernel']['workgroups']} workgroups x {dom['kernel']['threads']} threads)",
            "avg_ms": dom["ms"]}
    res = {"metric": METRIC, "value": tps, "unit": "tokens/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
           "ms_per_step": dt / a.steps * 1e3, "higher_is_better": True, "scaling": "weak",
           "vs_baseline": tps / c["publicado"] if c.get("publicado") else None, "dtype": "int8",
           "data": "synthetic: uniform random token ids, random-init weights (modelo.py init, seed 0)",
           "config": {"workload": c["nome"], "layers": c["L"], "d_model": c["D"], "heads": c["H"], "ffn": c["FF"],
                      "vocab": c["V"], "seq_len": c["T"], "batch": c["Bt"], "tokens_per_step": tokens, "block": c["BLK"],
                      "graph_launches": nlanc, "parallelism": "single GPU"},
           "loss_last_step": perda,
           "roofline": roof,
           "gemm_shapes": {k: {"M": v["M"], "N": v["N"], "K": v["K"], "mode": v["modo"], "ms": round(v["ms"], 5),
                               "TOPS": round(v["tops"], 2), "pct_i8_peak": round(100 * v["tops"] * 1e12 / PEAK_I8, 2),
                               "per_step": v["por_passo"], "kernel": v["kernel"]} for k, v in gem.items()},
           "gemm_ms_per_step_eager_sum": tot_gemm_ms}
    if not a.no_cpu:
        res["cpu_baseline"] = cpu_baseline(c, a.cpu_seconds)
        res["speedup_vs_cpu_baseline"] = tps / res["cpu_baseline"]["value"]
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
