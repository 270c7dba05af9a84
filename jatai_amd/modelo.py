"""The integer training step: the same composition of ops as the reference's `Modelo.passo`
(jatai_cuda/modelo.py:29-140) -- pre-norm decoder, RMSNorm without gain, causal ALiBi attention, ReLU^2 MLP,
byte vocabulary, Q/K/V in one matrix, SGD with momentum 7/8, lr = 2^-k and error feedback -- run on any backend
with the reference operator surface (OpsHip on the GPU; a CPU oracle in the tests and the CPU baseline).

`PassoGravado` captures one whole training step (forward, backward, optimizer: 522 launches op by op at L=12,
about 230 with the fusions below) as one hipGraph through torch.cuda.graph (reference: modelo.py:143-180).
Weights, momentum and residuals are updated in place by the kernels, every temporary lives in the graph's pool at
a fixed address, and the loss is computed inside the graph from the per-row integers (d_alvo, soma).
"""
import math
import os

import torch

from . import ops as O

R16 = os.environ.get("JATAI_RES16") == "1"     # 16-bit residual stream (modelo.py:26)


def inicial(g, linhas, fan_in, dev, emb=False):
    """Weight init: m = round(N(0,1) * 32) clamped to +-127, E = -round(log2(32 sqrt(fan_in))) (embedding: -5),
    drawn from the CPU generator g (modelo.py:16-19; Python's round on a float)."""
    e = -5 if emb else -int(round(math.log2(32 * math.sqrt(fan_in))))
    m = torch.round(torch.randn(linhas, fan_in, generator=g) * 32).clamp(-127, 127).to(torch.int8)
    return m.to(dev).contiguous(), torch.full((linhas, fan_in // O.BLK), e, dtype=torch.int8, device=dev)


def zeros_como(t):
    return torch.zeros_like(t[0]), torch.full_like(t[1], O.E_ZERO)


def perda_de(d_alvo, soma, ops=None):
    """Cross-entropy in nats from the integer softmax outputs: mean(d/256 + ln(s/4096)) in float64 (modelo.py:93);
    with `ops` (an ops object with `perda`), in its one launch instead of torch's six."""
    if ops is not None:
        return ops.perda(d_alvo, soma)
    return (d_alvo.double() / 256 + torch.log(soma.double() / 4096)).mean()


class Modelo:
    def __init__(self, V, D, H, FF, L, semente, dev, ops, reg, r16=None):
        self.V, self.D, self.H, self.FF, self.L, self.dev, self.ops, self.reg = V, D, H, FF, L, dev, ops, reg
        self.r16 = R16 if r16 is None else r16
        g = torch.Generator().manual_seed(semente)
        p = {"emb": inicial(g, V, D, dev, emb=True)}
        for l in range(L):
            q, k, v = inicial(g, D, D, dev), inicial(g, D, D, dev), inicial(g, D, D, dev)
            p[f"Wqkv{l}"] = (torch.cat([q[0], k[0], v[0]]).contiguous(), torch.cat([q[1], k[1], v[1]]).contiguous())
            p[f"Wo{l}"] = inicial(g, D, D, dev)
            p[f"Wup{l}"] = inicial(g, FF, D, dev)
            p[f"Wd{l}"] = inicial(g, D, FF, dev)
        p["out"] = inicial(g, V, D, dev)
        self.p = p
        self.mom = {n: zeros_como(t) for n, t in p.items()}
        self.res = {n: zeros_como(t) for n, t in p.items()}
        self.error_feedback = True
        self.estatisticas = False
        self.perda_inteira = False      # True: passo returns (d_alvo, soma) instead of the float64 loss
        # One fused optimizer launch over all tensors when the backend has it (OpsHip): the weight gradients are
        # written to persistent raw buffers whose addresses, with the weights', momenta's and residuals', sit in
        # a device table built once. Same results as momento then peso per tensor.
        self.otimizador_fundido = hasattr(ops, "otimizador")
        # Transposes of the weights and of the forward activations used by the backward, computed together in
        # batched launches right after the forward (same results as one transpoe per use).
        self.transpostas_em_lote = hasattr(ops, "transpoe_lote")
        # The weight-gradient GEMMs (K = tokens) deferred to the end of the backward and run together in grouped
        # launches (~10k tiles instead of 50 launches of 64-256 tiles); same results.
        self.dw_em_lote = hasattr(ops, "gemm_cru_lote")
        # momento + peso inside the grouped weight-gradient GEMM's epilogue, no gradient buffers (226 MB at config
        # 4). Off by default: the optimizer is bound by its own arithmetic, so the fusion saves little (a config-4
        # step 3.183 -> 3.162 ms, a config-5 step 34.49 -> 34.69 ms), and the separate launch keeps the GEMM's
        # own time measurable.
        self.otim_no_gemm = False
        # attention kernels that write their outputs quantized (quant(atencao), quant(atencao_back)): same results
        self.quant_na_atencao = hasattr(ops, "atencao_q")
        # in a training step, the forward attention's conversion pass also writes the backward's conversions of q, k,
        # v (a buffer per layer kept to the backward), whose conversion pass then reads only dO: same results. Off by
        # default: the backward's pass gets 2.6 us shorter and the forward's 1.95 us longer, and the backward kernels
        # that read those conversions lose 2.2 us, which they now fetch from HBM instead of from the cache the
        # backward's pass just wrote them to (config-4 step 3.132 -> 3.157 ms; config 5 34.23 either way)
        self.conversoes_salvas = False
        # the ReLU^2-backward GEMM also writes the transpose of its output (the next weight gradient's operand). Its
        # epilogue's transposed write is a serial tail of each workgroup, hidden by the other resident workgroups of
        # a large grid (config 5, 8192 workgroups: step 34.76 -> 34.62 ms) and about what the batched transpose it
        # replaces costs at one workgroup per CU (config 4: 2.9158 ms without it, 2.9151 with it). A workgroup
        # threshold (t_na_gemm_min_wg: None = 4 per CU of the device, 0 = always) can keep small grids batched.
        self.transposta_na_gemm = hasattr(ops, "gemm_relu2_back_t")
        self.t_na_gemm_min_wg = 0
        # the same for the FFN-up GEMM's ReLU^2 output a, whose transpose the weight gradient of the FFN-down layer
        # reads (training steps only; config 4 with both: 2.9149 ms, and the batched transposes of the step halved)
        self.transposta_na_relu2 = hasattr(ops, "gemm_relu2_t")
        self.t_na_relu2_min_wg = 0
        # the residual update of the backward, soma(gx, rms_back(...)), in one launch
        self.rms_soma = hasattr(ops, "rms_back_soma")
        # the R16 step's residual adds, soma16(x16, gemm(...)) and soma16(gx16, rms_back(...)), each with the INT8
        # copy para8 of its result (what the next RMSNorm or GEMMs read) in one launch
        self.soma16_fundida = hasattr(ops, "gemm_soma16") and hasattr(ops, "rms_back_soma16")
        # the loss in one launch of the library (float64 sums in another order than torch's mean: equal to 1e-15)
        self.perda_fundida = hasattr(ops, "perda")
        # measurement hook: stage name -> (before, after) callables run around that stage of the step
        # ("gradientes dos pesos": the grouped weight-gradient launch), e.g. to split a capture into three graphs
        # so the stage can be timed between replays as the step runs it
        self.marcas = {}
        self._gbuf, self._tabela, self._gbuf_compacto = None, None, None
        # the fused optimizer also writes transpoe(W) of every new weight but the embedding's (one workgroup per
        # 32 x 128 tile, jt_otimizador_t), which the next step's backward then reads instead of transposing the
        # weights again (BLK 32; the transposes are valid from the first fused update on, so the first step
        # transposes as before). A caller that changes weights outside the optimizer calls invalida_transpostas().
        self.transposta_no_otimizador = hasattr(ops, "tabela_otimizador") and O.BLK == 32 and all(
            t[0].shape[0] % 32 == 0 and t[0].shape[1] % 128 == 0 for t in self.p.values())
        self._pt, self._pt_validas, self._tabela_t, self._pt_lidas = None, False, None, False
        # the grouped weight-gradient launch writes the exponents of the fused optimizer's gradient buffers as row
        # and column vectors (OpsHip)
        self.grad_compacto = hasattr(ops, "gemm_cru_lote") and hasattr(ops, "otimizador")

    def _t_produtor(self, M, N, modo, min_wg):
        """Whether the ReLU^2 (modo 3) or ReLU^2-backward (modo 4) GEMM of M tokens x N columns, on a grid with a
        workgroup threshold of min_wg (None: 4 per CU of the device; 0: always), writes its transpose too. Only at
        BLK 32, where the GEMM's epilogue writes it (at BLK 128 a separate transpose per use would replace the batch)."""
        lib = getattr(self.ops, "lib", None)
        if O.BLK != 32:
            return False
        if min_wg == 0 or lib is None:
            return True
        if min_wg is None:
            min_wg = 4 * torch.cuda.get_device_properties(self.dev).multi_processor_count
        return (M // lib.jt_gemm_tile(M, N, modo)) * (N // 128) >= min_wg

    def _t_na_gemm(self, M, N):
        """Whether the ReLU^2-backward GEMM of M tokens x N columns writes its transpose too (see transposta_na_gemm)."""
        return self.transposta_na_gemm and self._t_produtor(M, N, 4, self.t_na_gemm_min_wg)

    def _t_na_relu2(self, M, N):
        """Whether the FFN-up GEMM of M tokens x N columns writes the transpose of its ReLU^2 output too."""
        return self.transposta_na_relu2 and self._t_produtor(M, N, 3, self.t_na_relu2_min_wg)

    def _otim_no_gemm(self):
        """Weight gradients straight into momento + peso in the grouped GEMM's epilogue (no gradient buffers)."""
        return self.otim_no_gemm and self.otimizador_fundido and self.dw_em_lote and hasattr(self.ops, "gemm_otim_lote")

    def _prepara_otimizador(self):
        # With the grouped weight-gradient launch the gradient buffers take the compact exponent form (a vector of
        # M + N: the exponent of (i, j) is RA_i + RB_j - 4), 2 bytes per value fewer written by the GEMM and read by
        # the optimizer; a per-GEMM launch writes one exponent per value.
        compacto = bool(self.dw_em_lote and self.grad_compacto)
        tw = self.transposta_no_otimizador
        if self._gbuf is None or self._gbuf_compacto != compacto or self._tabela_t != tw:
            ordem = ["out"] + [f"{w}{l}" for l in reversed(range(self.L)) for w in ("Wd", "Wup", "Wo", "Wqkv")] + ["emb"]
            fe = lambda t: (t.shape[0] + t.shape[1],) if compacto else t.shape
            self._gbuf = {n: (torch.empty(self.p[n][0].shape, dtype=torch.int32, device=self.dev),
                              torch.empty(fe(self.p[n][0]), dtype=torch.int16, device=self.dev)) for n in ordem}
            self._gbuf_compacto = compacto
            if tw and self._pt is None:         # transpoe(W) of each weight the backward reads: [N, M] blocked along M
                self._pt = {n: (torch.empty(self.p[n][0].shape[::-1], dtype=torch.int8, device=self.dev),
                                torch.empty(self.p[n][0].shape[1], self.p[n][0].shape[0] // O.BLK, dtype=torch.int8, device=self.dev))
                            for n in ordem if n != "emb"}
            self._tabela = self.ops.tabela_otimizador([(self._gbuf[n], self.mom[n], self.p[n], self.res[n],
                                                        self._pt.get(n) if tw else None) for n in ordem])
            self._tabela_t = tw
            self._pt_validas = False
        return self._gbuf

    def invalida_transpostas(self):
        """The weights changed outside the optimizer: the next eager step transposes them again, and a captured step
        (PassoGravado) rewrites the transposes it reads from the current weights before its next replay."""
        self._pt_validas = False

    def renova_transpostas(self):
        """transpoe(W) of the current weights into the buffers the fused optimizer writes (one batched launch)."""
        nomes = list(self._pt)
        for n, (Ym, YE) in zip(nomes, self.ops.transpoe_lote([self.p[n] for n in nomes])):
            self._pt[n][0].copy_(Ym)
            self._pt[n][1].copy_(YE)
        self._pt_validas = True

    def _st(self, nome, t, zeros_normais=False):
        if self.estatisticas:
            self.reg.estatistica(nome, t, zeros_normais)

    def passo(self, tok, alvo, k_lr=None):
        """Forward (+ backward and update when k_lr is given). Returns the loss as a tensor on the device."""
        ops, reg, p, r16 = self.ops, self.reg, self.p, self.r16
        s16 = r16 and self.soma16_fundida
        Bt, T = tok.shape
        x8 = None                   # R16: the INT8 copy of x16 when a fused launch wrote it

        def oito(x16):              # para8(x16), or the copy already written
            return x8 if x8 is not None else ops.para8(x16)
        tok, alvo = tok.reshape(-1).to(torch.int32).contiguous(), alvo.reshape(-1).to(torch.int32).contiguous()
        prontas = {}                # id(mantissas) -> transpose already written by its producer (or a batched launch)
        self._pt_lidas = False      # whether this step's backward reads the transposes the last fused update wrote
        with reg.trecho("forward"):
            with reg.trecho("embedding"):
                x = ops.embed(p["emb"], tok)
                if r16:
                    x16 = ops.para16(x)
            caches = []
            for l in range(self.L):
                with reg.trecho(f"camada {l}"):
                    with reg.trecho("atencao"):
                        n1, c1 = ops.rms(oito(x16) if r16 else x)
                        qkv = ops.gemm(n1, p[f"Wqkv{l}"])
                        sv = None
                        if self.quant_na_atencao and self.conversoes_salvas and k_lr is not None:
                            om, P, sv = ops.atencao_qs(qkv, Bt, T, self.H)
                        elif self.quant_na_atencao:
                            om, P = ops.atencao_q(qkv, Bt, T, self.H)
                        else:
                            oc, P = ops.atencao(qkv, Bt, T, self.H)
                            om = ops.quant(oc)
                        if s16:
                            x16, x8 = ops.gemm_soma16(om, p[f"Wo{l}"], x16)
                            x = x8 if self.estatisticas else None
                        elif r16:
                            x16 = ops.soma16(x16, ops.gemm(om, p[f"Wo{l}"]))
                            x = ops.para8(x16) if self.estatisticas else None
                        else:
                            x = ops.gemm_soma(om, p[f"Wo{l}"], x)
                        self._st(f"c{l}.qkv", qkv); self._st(f"c{l}.atencao_saida", om); self._st(f"c{l}.residuo1", x)
                    with reg.trecho("mlp"):
                        n2, c2 = ops.rms(oito(x16) if r16 else x)
                        if k_lr is not None and self._t_na_relu2(n2[0].shape[0], p[f"Wup{l}"][0].shape[0]):
                            h, a, ta = ops.gemm_relu2_t(n2, p[f"Wup{l}"])
                            prontas[id(a[0])] = ta
                        else:
                            h, a = ops.gemm_relu2(n2, p[f"Wup{l}"])
                        if s16:
                            x16, x8 = ops.gemm_soma16(a, p[f"Wd{l}"], x16)
                            x = x8 if self.estatisticas else None
                        elif r16:
                            x16 = ops.soma16(x16, ops.gemm(a, p[f"Wd{l}"]))
                            x = ops.para8(x16) if self.estatisticas else None
                        else:
                            x = ops.gemm_soma(a, p[f"Wd{l}"], x)
                        self._st(f"c{l}.relu2", a, zeros_normais=True); self._st(f"c{l}.residuo2", x)
                caches.append((n1, c1, qkv, P, om, n2, c2, h, a, sv))
            with reg.trecho("saida"):
                nf, cf = ops.rms(oito(x16) if r16 else x)
                logits = ops.gemm(nf, p["out"], cru=True)
                g, d_alvo, soma = ops.softmax_ce(logits, alvo)
        perda = (d_alvo, soma) if self.perda_inteira else perda_de(d_alvo, soma, ops if self.perda_fundida else None)
        if k_lr is None:
            return perda
        if self.transpostas_em_lote:
            with reg.trecho("transpostas"):
                pesos = [p[f"{w}{l}"] for l in range(self.L) for w in ("Wd", "Wup", "Wo", "Wqkv")] + [p["out"]]
                if self._pt_validas and self.otimizador_fundido and not self._otim_no_gemm():
                    for n, Y in self._pt.items():          # written by the last fused update
                        prontas[id(p[n][0])] = Y
                    pesos = []
                    self._pt_lidas = True
                ativ = [t for c in caches for t in (c[8], c[5], c[4], c[0]) if id(t[0]) not in prontas] + [nf]   # a, n2, om, n1
                for X, Y in zip(pesos + ativ, ops.transpoe_lote(pesos) + ops.transpoe_lote(ativ)):
                    prontas[id(X[0])] = Y

        def T_(X):
            Y = prontas.get(id(X[0]))
            return Y if Y is not None else ops.transpoe(X)
        grads = {}
        gb = self._prepara_otimizador() if self.otimizador_fundido and not self._otim_no_gemm() else None

        adiados = []

        def grad_w(n, X, Y):        # weight gradient T(X) . T(Y)^T, raw (into the persistent buffer when the optimizer is fused)
            if self.dw_em_lote:     # deferred: the transposes and the GEMMs run batched at the end of the backward
                adiados.append((n, X, Y))
                return None
            A, B = T_(X), T_(Y)
            return ops.gemm(A, B, cru=True, saida=gb[n]) if gb else ops.gemm(A, B, cru=True)
        with reg.trecho("backward"):
            with reg.trecho("saida"):
                grads["out"] = grad_w("out", g, nf)
                gx = ops.gemm(g, T_(p["out"]))
                gx = ops.rms_back(gx, nf, cf)
                self._st("grad_saida", gx)
                if r16:
                    gx16 = ops.para16(gx)
            for l in reversed(range(self.L)):
                n1, c1, qkv, P, om, n2, c2, h, a, sv = caches[l]
                with reg.trecho(f"camada {l}"):
                    with reg.trecho("mlp"):
                        grads[f"Wd{l}"] = grad_w(f"Wd{l}", gx, a)
                        if self._t_na_gemm(h[0].shape[0], h[0].shape[1]):
                            gh, tgh = ops.gemm_relu2_back_t(gx, T_(p[f"Wd{l}"]), h)
                            prontas[id(gh[0])] = tgh
                        else:
                            gh = ops.gemm_relu2_back(gx, T_(p[f"Wd{l}"]), h)
                        grads[f"Wup{l}"] = grad_w(f"Wup{l}", gh, n2)
                        gn = ops.gemm(gh, T_(p[f"Wup{l}"]))
                        if s16:
                            gx16, gx = ops.rms_back_soma16(gn, n2, c2, gx16)
                        elif r16:
                            gx16 = ops.soma16(gx16, ops.rms_back(gn, n2, c2))
                            gx = ops.para8(gx16)
                        else:
                            gx = ops.rms_back_soma(gn, n2, c2, gx) if self.rms_soma else ops.soma(gx, ops.rms_back(gn, n2, c2))
                        self._st(f"c{l}.grad_mlp", gh, zeros_normais=True)
                    with reg.trecho("atencao"):
                        grads[f"Wo{l}"] = grad_w(f"Wo{l}", gx, om)
                        go = ops.gemm(gx, T_(p[f"Wo{l}"]))
                        if sv is not None:
                            gq = ops.atencao_back_qs(go, qkv, P, sv, Bt, T, self.H)
                        elif self.quant_na_atencao:
                            gq = ops.atencao_back_q(go, qkv, P, Bt, T, self.H)
                        else:
                            gq = ops.quant(ops.atencao_back(go, qkv, P, Bt, T, self.H))
                        grads[f"Wqkv{l}"] = grad_w(f"Wqkv{l}", gq, n1)
                        gn = ops.gemm(gq, T_(p[f"Wqkv{l}"]))
                        if s16:
                            gx16, gx = ops.rms_back_soma16(gn, n1, c1, gx16)
                        elif r16:
                            gx16 = ops.soma16(gx16, ops.rms_back(gn, n1, c1))
                            gx = ops.para8(gx16)
                        else:
                            gx = ops.rms_back_soma(gn, n1, c1, gx) if self.rms_soma else ops.soma(gx, ops.rms_back(gn, n1, c1))
                        self._st(f"c{l}.grad_qkv", gq); self._st(f"c{l}.grad_residuo", gx)
            with reg.trecho("embedding"):
                um = ops.um_quente(tok, self.V)
                grads["emb"] = grad_w("emb", um, gx)
        if adiados and self.transpostas_em_lote:          # every transpose still missing, in one batched launch
            with reg.trecho("transpostas"):
                falta, vistos = [], set()
                for _, X, Y in adiados:
                    for Z in (X, Y):
                        if id(Z[0]) not in prontas and id(Z[0]) not in vistos:
                            vistos.add(id(Z[0]))
                            falta.append(Z)
                for Z, Zt in zip(falta, ops.transpoe_lote(falta)):
                    prontas[id(Z[0])] = Zt
        adiados = [(n, T_(X), T_(Y)) for n, X, Y in adiados]
        self._pt_validas = False                   # the weights change below; only jt_otimizador_t rewrites their transposes
        if adiados and self._otim_no_gemm():
            with reg.trecho("gradientes dos pesos + otimizador"):
                ops.gemm_otim_lote([(A, B, self.mom[n], self.p[n], self.res[n]) for n, A, B in adiados], k_lr, self.error_feedback)
            return perda
        if adiados:
            with reg.trecho("gradientes dos pesos"):
                marca = self.marcas.get("gradientes dos pesos")
                if marca:
                    marca[0]()
                for (n, _, _), G in zip(adiados, ops.gemm_cru_lote([(A, B, gb[n] if gb else None) for n, A, B in adiados],
                                                                   compacto=bool(gb) and self._gbuf_compacto)):
                    grads[n] = G
                if marca:
                    marca[1]()
        with reg.trecho("otimizador"):
            if self.otimizador_fundido:
                ops.otimizador(self._tabela, k_lr, self.error_feedback)
                self._pt_validas = bool(self._tabela_t)
                return perda
            for n, gr in grads.items():
                with reg.trecho(n):
                    self.mom[n] = ops.momento(gr, self.mom[n])
                    self.p[n], self.res[n] = ops.peso(self.p[n], self.mom[n], self.res[n], k_lr, self.error_feedback)
        return perda


class PassoGravado:
    """One training step captured as a hipGraph and replayed (modelo.py:143-180).

    Capture runs nothing (weights do not change while recording). Inputs go to fixed buffers with copy_ before
    each replay. The launch list of the capture (kid -> op, scope, inputs) is kept, so a device sentinel raised
    in a replay names the same op and scope as in eager mode. Format checks run once, at capture. The loss is
    computed inside the graph too: a call returns the graph's loss tensor, which the next replay overwrites.
    """

    def __init__(self, modelo, Bt, T, k_lr, corpus=None):
        self.m, self.reg, self.k_lr = modelo, modelo.reg, k_lr
        lib = modelo.ops.lib
        # int32, the kernels' token type: the replay's copy_ converts, and the graph holds no conversion
        self.tok = torch.zeros(Bt, T, dtype=torch.int32, device=modelo.dev)
        self.alvo = torch.zeros(Bt, T, dtype=torch.int32, device=modelo.dev)
        # with a device-resident corpus (jatai_amd.dados.Corpus) the graph starts with the window gather, and a
        # step's only input is its Bt window starts
        self.corpus, self.Bt, self.T = corpus, Bt, T
        self.ini = torch.zeros(Bt, dtype=torch.int64, device=modelo.dev) if corpus is not None else None
        self.grafo = torch.cuda.CUDAGraph()
        est, vig, pi = modelo.estatisticas, self.reg.vigiar, modelo.perda_inteira
        modelo.estatisticas, self.reg.vigiar, modelo.perda_inteira = False, False, True
        if modelo.otimizador_fundido and not modelo._otim_no_gemm():
            modelo._prepara_otimizador()          # buffers and the device table exist before capture
        torch.cuda.synchronize()
        self.reg.lancamentos = []
        try:
            with torch.cuda.graph(self.grafo):
                lib.jt_stream(torch.cuda.current_stream().cuda_stream)
                if corpus is not None:
                    with self.reg.trecho("dados"):
                        corpus.janelas(self.ini, T, self.tok, self.alvo)
                self.d_alvo, self.soma = modelo.passo(self.tok, self.alvo, k_lr=k_lr)
                self.perda = perda_de(self.d_alvo, self.soma, modelo.ops if modelo.perda_fundida else None)     # in the graph, as modelo.py:170 captures passo's loss
        finally:
            lib.jt_stream(None)
            modelo.estatisticas, self.reg.vigiar, modelo.perda_inteira = est, vig, pi
        self.lancamentos = list(self.reg.lancamentos)
        # the captured backward reads the weights' transposes from the buffers the fused update writes (at capture
        # they held the transposes of the current weights); weights changed since outside the graph's own update
        # (invalida_transpostas) need them rewritten before the next replay
        self.le_transpostas = modelo._pt_lidas
        self.reg.info(f"passo gravado num hipGraph: {len(self.lancamentos)} lancamentos", lancamentos=len(self.lancamentos))

    def _transpostas_em_dia(self):
        if self.le_transpostas and not self.m._pt_validas:
            self.reg.lancamentos = list(self.reg.lancamentos)    # never append to the graph's own list
            self.m.renova_transpostas()
            self.reg.confere_device()    # a sentinel of those launches is read while the step's list still names them

    def __call__(self, tok, alvo):
        if self.corpus is not None:
            raise RuntimeError("this graph reads its tokens from its corpus: call de_corpus(gerador)")
        self._transpostas_em_dia()
        self.tok.copy_(tok)
        self.alvo.copy_(alvo)
        self.reg.lancamentos = self.lancamentos
        self.grafo.replay()
        return self.perda

    def de_corpus(self, gerador):
        """One step on the batch that jatai_amd.dados.lote(dados, gerador, Bt, T) would draw: the Bt starts go to
        the device (64 bytes at Bt = 8) and the graph's first node writes the windows into its token buffers."""
        self._transpostas_em_dia()
        self.ini.copy_(self.corpus.inicios(gerador, self.Bt, self.T))
        self.reg.lancamentos = self.lancamentos
        self.grafo.replay()
        return self.perda
