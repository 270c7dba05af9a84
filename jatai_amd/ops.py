"""Operator surface of the Jatai INT8 training hot path on MI355X.

`OpsHip` has the methods, arguments, return structure, shape guards and error behaviour of the reference's
`OpsCuda` (jatai_cuda/ops.py:294-515): model code written against `OpsCuda` (modelo.py, treino_cuda.py,
teste_ops.py) runs unchanged with `OpsHip`. Each method checks formats on the host, allocates its outputs
with torch on the caller's device, and launches one hand-written gfx950 kernel through the C ABI of
`libjatai.so` (include/jatai.h) via ctypes.

Module globals read by callers, as in the reference: BLK (block size, 32 or 128; the reference fixes 128,
ops.py:17), E_ZERO, GA, ATENCAO_LIMITE (attention-backward bound variant, ops.py:23), g_rms.

There is no CPU fallback: if libjatai.so is missing or fails to load, constructing OpsHip raises.
"""
import ctypes
import math
import os

import torch

BLK = 128
E_ZERO = -127
GA = 4
ATENCAO_LIMITE = False
# attention through the workspace entry points (jt_atencao_ws): same outputs, faster at head width 64; False runs
# the reference ABI's jt_atencao
ATENCAO_WS = True
AQUI = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(AQUI, "libjatai.so")

FUNCOES = ("jt_gemm", "jt_gemm_f", "jt_quant", "jt_soma", "jt_relu2", "jt_relu2_back", "jt_momento", "jt_peso", "jt_transpoe",
           "jt_embed", "jt_um_quente", "jt_rms", "jt_rms_back", "jt_atencao", "jt_atencao_back", "jt_softmax_ce", "jt_erro_le",
           "jt_erro_limpa", "jt_sincroniza", "jt_para16", "jt_para8", "jt_soma16", "jt_res_estocastico", "jt_bloco",
           "jt_bloco_atual", "jt_otimizador", "jt_tab_otim_bytes", "jt_transpoe_lote", "jt_entrada_t_bytes", "jt_gemm_divisoes",
           "jt_atencao_ws", "jt_atencao_back_ws", "jt_gemm_lote", "jt_entrada_g_bytes",
           "jt_gemm_otim_lote", "jt_entrada_go_bytes", "jt_atencao_ws_q", "jt_atencao_back_ws_q",
           "jt_rms_back_soma", "jt_perda", "jt_gemm_tile", "jt_gemm_soma16", "jt_rms_back_soma16", "jt_atencao_ws_qs",
           "jt_atencao_back_ws_qs", "jt_janelas", "jt_otimizador_t")
VOIDS = ("jt_stream", "jt_gemm_split", "jt_gemm_bm", "jt_atencao_linhas", "jt_atencao_mfma")


def g_rms(D):
    """(G of the RMSNorm, G of its backward) for width D at the current BLK (ops.py:28-30)."""
    nb = D // BLK
    return 2 * ((8 - int(math.log2(nb))) // 2), 14 - int(math.log2(D))


def carrega_lib(caminho=LIB):
    """Load libjatai.so after torch, so the library binds to the HIP runtime torch already loaded (both carry
    the soname libamdhip64.so.7): streams from torch.cuda are then valid handles for jt_stream."""
    if not os.path.exists(caminho):
        raise RuntimeError(f"libjatai.so not built ({caminho}); run `python -m jatai_amd.build` or __graft_entry__.build()")
    lib = ctypes.CDLL(caminho)
    for f in FUNCOES:
        getattr(lib, f).restype = ctypes.c_int
    for f in VOIDS:
        getattr(lib, f).restype = None
    lib.jt_stream.argtypes = [ctypes.c_void_p]
    lib.jt_erro_le.argtypes = [ctypes.c_void_p]
    lib.jt_atencao_ws_bytes.restype = ctypes.c_longlong
    lib.jt_atencao_back_ws_bytes.restype = ctypes.c_longlong
    lib.jt_atencao_salvo_bytes.restype = ctypes.c_longlong
    return lib


class OpsHip:
    nome = "hip"
    lib_global = None

    def __init__(self, reg):
        self.reg = reg
        self.lib = carrega_lib()
        reg.lib = self.lib
        if self.lib.jt_erro_limpa() != 0:
            raise RuntimeError("libjatai: could not clear the device error record (no usable GPU?)")
        if os.environ.get("JATAI_RES_EST") == "1":      # stochastic residual rounding in gemm_soma (ops.py:308-309)
            rc = self.lib.jt_res_estocastico(1)
            if rc != 0:
                raise RuntimeError(f"JATAI_RES_EST=1: jt_res_estocastico failed ({rc})")
        self._blk = None
        OpsHip.lib_global = self.lib

    @staticmethod
    def _a(x):
        if torch.is_tensor(x):
            return ctypes.c_void_p(x.data_ptr()) if x.numel() else ctypes.c_void_p(0)
        if x is None:
            return ctypes.c_void_p(0)
        return ctypes.c_longlong(x) if isinstance(x, int) and abs(x) > 2**31 - 1 else ctypes.c_int(x)

    def _lanca(self, op, fn, args, entradas, forma, longos=()):
        if self._blk != BLK:
            self.reg.exige(self.lib.jt_bloco(BLK) == 0, f"BLK={BLK} not supported (32 or 128)")
            self._blk = BLK
        kid = self.reg.registra(op, entradas, forma)
        conv = [ctypes.c_longlong(a) if i in longos else self._a(a) for i, a in enumerate(args)]
        r = getattr(self.lib, fn)(*conv, ctypes.c_int(kid))
        self.reg.depois(kid, r)

    def _novo_bloco(self, R, C, dev):
        return torch.empty(R, C, dtype=torch.int8, device=dev), torch.empty(R, C // BLK, dtype=torch.int8, device=dev)

    # ---------------------------------------------------------------- GEMM family (ops.py:329-372)
    def _formas_gemm(self, op, a, b):
        M, K = a.shape
        N = b.shape[0]
        self.reg.exige(b.shape[1] == K, f"{op}: K diferente, A {tuple(a.shape)} x B {tuple(b.shape)}")
        # K <= 4096 as the reference (ops.py:336-337); beyond it (up to 65536) the kernel walks K in chunks of 2048
        # values of shift tables, reads the exponent rows with 16-byte loads and so needs K / BLK to be a multiple of 16
        self.reg.exige(M % 32 == 0 and N % 128 == 0 and K % BLK == 0 and 0 < K and (K <= 4096 or (K <= 65536 and (K // BLK) % 16 == 0)),
                       f"{op}: M multiplo de 32, N de 128, K de {BLK} e K <= 4096 (ou K <= 65536 com K/{BLK} multiplo de 16) "
                       f"(M={M}, N={N}, K={K})")
        return M, N, K

    def gemm(self, A, B, cru=False, saida=None):
        """`saida`: optional preallocated raw output (int32 [M, N], int16 [M, N]) for cru=True."""
        reg = self.reg
        reg.confere_bloco("A", A); reg.confere_bloco("B", B)
        (a, ea), (b, eb) = A, B
        M, N, K = self._formas_gemm("gemm", a, b)
        if cru:
            if saida is not None:
                reg.exige(saida[0].dtype == torch.int32 and saida[1].dtype == torch.int16 and tuple(saida[0].shape) == (M, N)
                          and tuple(saida[1].shape) == (M, N) and saida[0].is_contiguous() and saida[1].is_contiguous(),
                          f"gemm: saida deve ser (int32, int16) contiguos de forma {(M, N)}")
                C = saida
            else:
                C = (torch.empty(M, N, dtype=torch.int32, device=a.device), torch.empty(M, N, dtype=torch.int16, device=a.device))
            self._lanca("gemm_cru", "jt_gemm", (a, ea, b, eb, None, None, C[0], C[1], M, N, K, 1), dict(A=a, EA=ea, B=b, EB=eb), (M, N))
        else:
            C = self._novo_bloco(M, N, a.device)
            self._lanca("gemm", "jt_gemm", (a, ea, b, eb, C[0], C[1], None, None, M, N, K, 0), dict(A=a, EA=ea, B=b, EB=eb), (M, N))
        return C

    # no reference counterpart: many raw GEMMs sharing K in one launch (64 per launch)
    def gemm_cru_lote(self, pares, compacto=False):
        """[gemm(A, B, cru=True, saida=S) for (A, B, S) in pares]; S may be None. Launch ids are consecutive.
        compacto: each S[1] is an int16 vector of M + N holding the exponents as RA_i (first M) and RB_j - 4 (last N),
        whose sum is the exponent of (i, j) -- the form the fused optimizer reads."""
        if not pares:
            return []
        if self._blk != BLK:
            self.reg.exige(self.lib.jt_bloco(BLK) == 0, f"BLK={BLK} not supported (32 or 128)")
            self._blk = BLK
        self.reg.exige(self.lib.jt_entrada_g_bytes() == 64, "gemm_cru_lote: tamanho de entrada inesperado")
        tab = (ctypes.c_longlong * (8 * len(pares)))()
        saidas, kid0 = [], None
        for i, (A, B, S) in enumerate(pares):
            self.reg.confere_bloco("A", A); self.reg.confere_bloco("B", B)
            (a, ea), (b, eb) = A, B
            M, N, K = self._formas_gemm("gemm", a, b)
            fe = (M + N,) if compacto else (M, N)
            if S is None:
                S = (torch.empty(M, N, dtype=torch.int32, device=a.device), torch.empty(fe, dtype=torch.int16, device=a.device))
            self.reg.exige(S[0].dtype == torch.int32 and S[1].dtype == torch.int16 and tuple(S[0].shape) == (M, N)
                           and tuple(S[1].shape) == fe and S[0].is_contiguous() and S[1].is_contiguous(),
                           f"gemm_cru_lote: saida deve ser (int32 {(M, N)}, int16 {fe}) contiguos")
            saidas.append(S)
            kid = self.reg.registra("gemm_cru", dict(A=a, EA=ea, B=b, EB=eb), (M, N), tempo=(i == 0))
            kid0 = kid if kid0 is None else kid0
            tab[8 * i:8 * i + 8] = [a.data_ptr(), ea.data_ptr(), b.data_ptr(), eb.data_ptr(), S[0].data_ptr(), S[1].data_ptr(),
                                    (N << 32) | M, (int(compacto) << 32) | K]
        r = self.lib.jt_gemm_lote(ctypes.cast(tab, ctypes.c_void_p), ctypes.c_int(len(pares)), ctypes.c_int(kid0))
        self.reg.depois(kid0, r)
        return saidas

    # no reference counterpart: weight-gradient GEMMs with momento + peso in the epilogue (32 per launch)
    def gemm_otim_lote(self, itens, k, ef):
        """For (A, B, Mom, W, R) in itens: momento(gemm(A, B, cru=True), Mom) then peso(W, Mom, R, k, ef), in place,
        without storing the gradient. Launch ids are consecutive, one per item."""
        if not itens:
            return
        if self._blk != BLK:
            self.reg.exige(self.lib.jt_bloco(BLK) == 0, f"BLK={BLK} not supported (32 or 128)")
            self._blk = BLK
        self.reg.exige(self.lib.jt_entrada_go_bytes() == 96, "gemm_otim_lote: tamanho de entrada inesperado")
        tab = (ctypes.c_longlong * (12 * len(itens)))()
        kid0 = None
        for i, (A, B, Mom, W, R) in enumerate(itens):
            self.reg.confere_bloco("A", A); self.reg.confere_bloco("B", B)
            for n_, t in (("momento", Mom), ("W", W), ("residuo", R)):
                self.reg.confere_bloco(n_, t)
            (a, ea), (b, eb) = A, B
            M, N, K = self._formas_gemm("gemm", a, b)
            self.reg.exige(all(tuple(t[0].shape) == (M, N) for t in (Mom, W, R)), f"gemm_otim_lote: peso de forma diferente de {(M, N)}")
            kid = self.reg.registra("gemm_cru+otimizador", dict(A=a, EA=ea, B=b, EB=eb), (M, N), tempo=(i == 0))
            kid0 = kid if kid0 is None else kid0
            tab[12 * i:12 * i + 12] = [a.data_ptr(), ea.data_ptr(), b.data_ptr(), eb.data_ptr(), Mom[0].data_ptr(), Mom[1].data_ptr(),
                                       W[0].data_ptr(), W[1].data_ptr(), R[0].data_ptr(), R[1].data_ptr(), (N << 32) | M, K]
        r = self.lib.jt_gemm_otim_lote(ctypes.cast(tab, ctypes.c_void_p), ctypes.c_int(len(itens)), ctypes.c_int(k), ctypes.c_int(int(ef)),
                                       ctypes.c_int(kid0))
        self.reg.depois(kid0, r)

    def _gemm_fundida(self, op, modo, A, B, X=None, saida2=False):
        reg = self.reg
        reg.confere_bloco("A", A); reg.confere_bloco("B", B)
        (a, ea), (b, eb) = A, B
        M, N, K = self._formas_gemm(op, a, b)
        ent = dict(A=a, EA=ea, B=b, EB=eb)
        if X is not None:
            reg.confere_bloco("X", X)
            reg.exige(tuple(X[0].shape) == (M, N), f"{op}: X com forma {tuple(X[0].shape)}, esperado {(M, N)}")
            ent.update(X=X[0], XE=X[1])
        C = self._novo_bloco(M, N, a.device)
        C2 = self._novo_bloco(M, N, a.device) if saida2 else (None, None)
        self._lanca(op, "jt_gemm_f", (a, ea, b, eb, C[0], C[1], None, None, X[0] if X is not None else None,
                                      X[1] if X is not None else None, C2[0], C2[1], M, N, K, modo), ent, (M, N))
        return (C, C2) if saida2 else C

    def gemm_soma(self, A, B, X):
        return self._gemm_fundida("gemm_soma", 2, A, B, X=X)

    def gemm_relu2(self, A, B):
        return self._gemm_fundida("gemm_relu2", 3, A, B, saida2=True)

    # no reference counterpart: (gemm_relu2_back(A, B, Hh), its transpose) from one launch at BLK = 32
    def gemm_relu2_back_t(self, A, B, Hh):
        if BLK != 32:
            G = self.gemm_relu2_back(A, B, Hh)
            return G, self.transpoe(G)
        reg = self.reg
        reg.confere_bloco("A", A); reg.confere_bloco("B", B); reg.confere_bloco("X", Hh)
        (a, ea), (b, eb) = A, B
        M, N, K = self._formas_gemm("gemm_relu2_back", a, b)
        reg.exige(tuple(Hh[0].shape) == (M, N), f"gemm_relu2_back: X com forma {tuple(Hh[0].shape)}, esperado {(M, N)}")
        C, Ct = self._novo_bloco(M, N, a.device), self._novo_bloco(N, M, a.device)
        self._lanca("gemm_relu2_back+transpoe", "jt_gemm_f", (a, ea, b, eb, C[0], C[1], None, None, Hh[0], Hh[1], Ct[0], Ct[1], M, N, K, 4),
                    dict(A=a, EA=ea, B=b, EB=eb, X=Hh[0], XE=Hh[1]), (M, N))
        return C, Ct

    # no reference counterpart: (gemm_relu2(A, B), transpoe of its ReLU^2 output) from one launch at BLK = 32
    def gemm_relu2_t(self, A, B):
        if BLK != 32:
            h, a = self.gemm_relu2(A, B)
            return h, a, self.transpoe(a)
        reg = self.reg
        reg.confere_bloco("A", A); reg.confere_bloco("B", B)
        (a, ea), (b, eb) = A, B
        M, N, K = self._formas_gemm("gemm_relu2", a, b)
        Hh, Aa, At = self._novo_bloco(M, N, a.device), self._novo_bloco(M, N, a.device), self._novo_bloco(N, M, a.device)
        self._lanca("gemm_relu2+transpoe", "jt_gemm_f", (a, ea, b, eb, Hh[0], Hh[1], At[0], At[1], None, None, Aa[0], Aa[1], M, N, K, 3),
                    dict(A=a, EA=ea, B=b, EB=eb), (M, N))
        return Hh, Aa, At

    def gemm_relu2_back(self, A, B, Hh):
        return self._gemm_fundida("gemm_relu2_back", 4, A, B, X=Hh)

    # ---------------------------------------------------------------- re-blocking and element-wise (ops.py:374-432)
    def transpoe(self, X):
        self.reg.confere_bloco("X", X)
        m, E = X
        R, C = m.shape
        self.reg.exige(R % 128 == 0 and C % 64 == 0, f"transpoe: linhas {R} nao multiplo de 128 ou colunas {C} nao multiplo de 64")
        Y = self._novo_bloco(C, R, m.device)
        self._lanca("transpoe", "jt_transpoe", (m, E, Y[0], Y[1], R, C), dict(X=m, EX=E), (C, R))
        return Y

    # no reference counterpart: many transposes in one launch (64 tensors per launch)
    def transpoe_lote(self, Xs):
        """[transpoe(X) for X in Xs], computed by batched launches; launch ids are consecutive, one per tensor."""
        if not Xs:
            return []
        if self._blk != BLK:
            self.reg.exige(self.lib.jt_bloco(BLK) == 0, f"BLK={BLK} not supported (32 or 128)")
            self._blk = BLK
        self.reg.exige(self.lib.jt_entrada_t_bytes() == 40, "transpoe_lote: tamanho de entrada inesperado")
        Ys, tab = [], (ctypes.c_longlong * (5 * len(Xs)))()
        kid0 = None
        for i, X in enumerate(Xs):
            self.reg.confere_bloco("X", X)
            m, E = X
            R, C = m.shape
            self.reg.exige(R % 128 == 0 and C % 64 == 0, f"transpoe: linhas {R} nao multiplo de 128 ou colunas {C} nao multiplo de 64")
            Y = self._novo_bloco(C, R, m.device)
            Ys.append(Y)
            kid = self.reg.registra("transpoe", dict(X=m, EX=E), (C, R), tempo=(i == 0))
            kid0 = kid if kid0 is None else kid0
            self.reg.exige(kid == kid0 + i, "transpoe_lote: ids de lancamento nao consecutivos")
            tab[5 * i:5 * i + 5] = [m.data_ptr(), E.data_ptr(), Y[0].data_ptr(), Y[1].data_ptr(), (C << 32) | R]
        r = self.lib.jt_transpoe_lote(ctypes.cast(tab, ctypes.c_void_p), ctypes.c_int(len(Xs)), ctypes.c_int(kid0))
        self.reg.depois(kid0, r)
        return Ys

    def de_f32(self, x):
        """float32 [R, C] to a block tensor: each value split exactly into an integer mantissa and an exponent
        (frexp: x = v 2^e, |v| < 2^24, an int32 / int16 raw tensor), then the spec's quant of that raw tensor
        (ops.py:58-72). Integer-only after the exact split; the data path of BASELINE configs 2 and 3 (fp32 N(0, 1)
        activations, N(0, 0.02) weights). Finite inputs only."""
        self.reg.exige(x.dtype == torch.float32 and x.dim() == 2 and x.is_cuda, "de_f32: espera float32 [R, C] na GPU")
        self.reg.exige(bool(torch.isfinite(x).all()), "de_f32: valores nao finitos")
        m, e = torch.frexp(x)
        v = (m * float(1 << 24)).to(torch.int32)
        return self.quant((v.contiguous(), (e - 24).to(torch.int16).contiguous()))

    def quant(self, Cc):
        self.reg.confere_cru("C", Cc)
        acc, e = Cc
        R, C = acc.shape
        self.reg.exige(C % BLK == 0, f"quant: colunas {C} nao multiplo de {BLK}")
        Y = self._novo_bloco(R, C, acc.device)
        self._lanca("quant", "jt_quant", (acc, e, Y[0], Y[1], R * C // BLK), dict(acc=acc, e=e), (R, C), longos=(4,))
        return Y

    def _elem(self, op, fn, ins, nomes):
        for n, t in zip(nomes, ins):
            self.reg.confere_bloco(n, t)
        m0 = ins[0][0]
        for n, t in zip(nomes[1:], ins[1:]):
            self.reg.exige(t[0].shape == m0.shape, f"{op}: '{n}' com forma {tuple(t[0].shape)}, esperado {tuple(m0.shape)}")
        Y = self._novo_bloco(*m0.shape, m0.device)
        args = [x for t in ins for x in t] + [Y[0], Y[1], m0.numel() // BLK]
        ent = {f"{n}{s}": x for n, t in zip(nomes, ins) for s, x in zip(("", "E"), t)}
        self._lanca(op, fn, args, ent, tuple(m0.shape), longos=(len(args) - 1,))
        return Y

    def soma(self, X, Y):
        return self._elem("soma", "jt_soma", (X, Y), ("x", "y"))

    # ---- 16-bit residual stream: (int16 mantissa, int8 exponent per block) (ops.py:406-426)
    def _r16(self, op, fn, args, ent, forma, saida16):
        m0 = args[0]
        R, C = forma
        Y = (torch.empty(R, C, dtype=torch.int16 if saida16 else torch.int8, device=m0.device),
             torch.empty(R, C // BLK, dtype=torch.int8, device=m0.device))
        a = list(args) + [Y[0], Y[1], R * C // BLK]
        self._lanca(op, fn, a, ent, forma, longos=(len(a) - 1,))
        return Y

    def para16(self, X):
        self.reg.confere_bloco("x", X)
        return self._r16("para16", "jt_para16", X, dict(x=X[0], xE=X[1]), tuple(X[0].shape), True)

    def para8(self, X16):
        self.reg.confere_r16("x16", X16)
        return self._r16("para8", "jt_para8", X16, dict(x16=X16[0], xE=X16[1]), tuple(X16[0].shape), False)

    def soma16(self, X16, Y):
        self.reg.confere_r16("x16", X16)
        self.reg.confere_bloco("y", Y)
        self.reg.exige(tuple(Y[0].shape) == tuple(X16[0].shape), f"soma16: formas {tuple(X16[0].shape)} e {tuple(Y[0].shape)}")
        return self._r16("soma16", "jt_soma16", (*X16, *Y), dict(x16=X16[0], y=Y[0]), tuple(X16[0].shape), True)

    # no reference counterpart: (soma16(X16, gemm(A, B)), para8 of it) from one launch -- the R16 step's residual add
    # and the INT8 copy its next RMSNorm reads; the same bits as the three ops in turn
    def gemm_soma16(self, A, B, X16):
        reg = self.reg
        reg.confere_bloco("A", A); reg.confere_bloco("B", B); reg.confere_r16("x16", X16)
        (a, ea), (b, eb) = A, B
        M, N, K = self._formas_gemm("gemm_soma16", a, b)
        reg.exige(tuple(X16[0].shape) == (M, N), f"gemm_soma16: x16 com forma {tuple(X16[0].shape)}, esperado {(M, N)}")
        Z = (torch.empty(M, N, dtype=torch.int16, device=a.device), torch.empty(M, N // BLK, dtype=torch.int8, device=a.device))
        Y = self._novo_bloco(M, N, a.device)
        if self._blk != BLK:
            self.reg.exige(self.lib.jt_bloco(BLK) == 0, f"BLK={BLK} not supported (32 or 128)")
            self._blk = BLK
        # launch ids: kid the GEMM, kid + 1 its soma16 stage, kid + 2 its para8 stage (a device event names its stage)
        kid = self.reg.registra("gemm_soma16", dict(A=a, EA=ea, B=b, EB=eb, x16=X16[0], xE=X16[1]), (M, N))
        self.reg.registra("soma16", dict(x16=X16[0], xE=X16[1]), (M, N), tempo=False)
        self.reg.registra("para8", dict(), (M, N), tempo=False)
        r = self.lib.jt_gemm_soma16(*[self._a(t) for t in (a, ea, b, eb, X16[0], X16[1], Z[0], Z[1], Y[0], Y[1])], M, N, K,
                                    ctypes.c_int(kid))
        self.reg.depois(kid, r)
        return Z, Y

    def relu2(self, Hh):
        return self._elem("relu2", "jt_relu2", (Hh,), ("h",))

    def relu2_back(self, Gg, Hh):
        return self._elem("relu2_back", "jt_relu2_back", (Gg, Hh), ("g", "h"))

    def embed(self, W, tok):
        self.reg.confere_bloco("W", W)
        m, E = W
        V, D = m.shape
        M = tok.numel()
        X = self._novo_bloco(M, D, m.device)
        self._lanca("embed", "jt_embed", (m, E, tok, X[0], X[1], M, D, V), dict(W=m, tok=tok), (M, D))
        return X

    def janelas(self, corpus, ini, T, tok=None, alvo=None):
        """Training windows from a device-resident byte corpus (treino_int8_gpu/treino.py:41-44 draws them on the
        host): tok[b, t] = corpus[ini[b] + t], alvo[b, t] = corpus[ini[b] + t + 1], int32. corpus: uint8 [n] on the
        device; ini: int64 [Bt] on the device. tok and alvo ([Bt, T] int32) are written in place when given."""
        Bt, n = ini.numel(), corpus.numel()
        if tok is None:
            tok = torch.empty(Bt, T, dtype=torch.int32, device=corpus.device)
        if alvo is None:
            alvo = torch.empty(Bt, T, dtype=torch.int32, device=corpus.device)
        self.reg.exige(corpus.dtype == torch.uint8 and ini.dtype == torch.int64, "janelas: corpus uint8 and ini int64")
        self.reg.exige(tuple(tok.shape) == (Bt, T) and tuple(alvo.shape) == (Bt, T) and tok.dtype == torch.int32
                       and alvo.dtype == torch.int32, f"janelas: tok and alvo must be int32 [{Bt}, {T}]")
        self._lanca("janelas", "jt_janelas", (corpus, n, ini, tok, alvo, Bt, T), dict(ini=ini), (Bt, T), longos=(1,))
        return tok, alvo

    def um_quente(self, tok, V):
        M = tok.numel()
        U = self._novo_bloco(M, V, tok.device)
        self._lanca("um_quente", "jt_um_quente", (tok, U[0], U[1], M, V), dict(tok=tok), (M, V))
        return U

    # ---------------------------------------------------------------- rows (ops.py:449-502)
    def rms(self, X):
        self.reg.confere_bloco("x", X)
        m, E = X
        M, D = m.shape
        self.reg.exige(D <= 1024, f"rms: D={D} > 1024 nao suportado")
        G, _ = g_rms(D)
        Y = self._novo_bloco(M, D, m.device)
        r = torch.empty(M, dtype=torch.int32, device=m.device)
        emax = torch.empty(M, dtype=torch.int32, device=m.device)
        self._lanca("rms", "jt_rms", (m, E, Y[0], Y[1], r, emax, M, D, int(math.log2(D)), G), dict(x=m, xE=E), (M, D))
        return Y, (r, emax)

    def rms_back(self, Gg, Y, cache):
        self.reg.confere_bloco("g", Gg); self.reg.confere_bloco("y", Y)
        (g, gE), (y, yE) = Gg, Y
        M, D = g.shape
        self.reg.exige(D <= 1024, f"rms_back: D={D} > 1024 nao suportado")
        G, GB = g_rms(D)
        O = self._novo_bloco(M, D, g.device)
        self._lanca("rms_back", "jt_rms_back", (g, gE, y, yE, cache[0], cache[1], O[0], O[1], M, D, int(math.log2(D)), G, GB),
                    dict(g=g, gE=gE, y=y, yE=yE, r=cache[0], emax=cache[1]), (M, D))
        return O

    # no reference counterpart: soma(X, rms_back(Gg, Y, cache)) in one launch; launch ids for both parts
    def rms_back_soma(self, Gg, Y, cache, X):
        self.reg.confere_bloco("g", Gg); self.reg.confere_bloco("y", Y); self.reg.confere_bloco("x", X)
        (g, gE), (y, yE), (x, xE) = Gg, Y, X
        M, D = g.shape
        self.reg.exige(tuple(x.shape) == (M, D), f"rms_back_soma: x com forma {tuple(x.shape)}, esperado {(M, D)}")
        G, GB = g_rms(D)
        O = self._novo_bloco(M, D, g.device)
        if self._blk != BLK:
            self.reg.exige(self.lib.jt_bloco(BLK) == 0, f"BLK={BLK} not supported (32 or 128)")
            self._blk = BLK
        kid = self.reg.registra("rms_back", dict(g=g, gE=gE, y=y, yE=yE, r=cache[0], emax=cache[1]), (M, D))
        self.reg.registra("soma", dict(x=x, xE=xE), (M, D), tempo=False)
        r = self.lib.jt_rms_back_soma(*[self._a(t) for t in (g, gE, y, yE, cache[0], cache[1], x, xE, O[0], O[1])], M, D, int(math.log2(D)),
                                      G, GB, ctypes.c_int(kid))
        self.reg.depois(kid, r)
        return O

    # no reference counterpart: (soma16(X16, rms_back(g, y, cache)), para8 of it) in one launch -- the R16 backward's
    # residual update and the INT8 copy the next GEMMs read; launch ids: rms_back, soma16, para8
    def rms_back_soma16(self, Gg, Y, cache, X16):
        self.reg.confere_bloco("g", Gg); self.reg.confere_bloco("y", Y); self.reg.confere_r16("x16", X16)
        (g, gE), (y, yE), (x, xE) = Gg, Y, X16
        M, D = g.shape
        self.reg.exige(tuple(x.shape) == (M, D), f"rms_back_soma16: x16 com forma {tuple(x.shape)}, esperado {(M, D)}")
        G, GB = g_rms(D)
        Z = (torch.empty(M, D, dtype=torch.int16, device=g.device), torch.empty(M, D // BLK, dtype=torch.int8, device=g.device))
        O = self._novo_bloco(M, D, g.device)
        if self._blk != BLK:
            self.reg.exige(self.lib.jt_bloco(BLK) == 0, f"BLK={BLK} not supported (32 or 128)")
            self._blk = BLK
        kid = self.reg.registra("rms_back", dict(g=g, gE=gE, y=y, yE=yE, r=cache[0], emax=cache[1]), (M, D))
        self.reg.registra("soma16", dict(x16=x, xE=xE), (M, D), tempo=False)
        self.reg.registra("para8", dict(), (M, D), tempo=False)
        r = self.lib.jt_rms_back_soma16(*[self._a(t) for t in (g, gE, y, yE, cache[0], cache[1], x, xE, Z[0], Z[1], O[0], O[1])], M, D,
                                        int(math.log2(D)), G, GB, ctypes.c_int(kid))
        self.reg.depois(kid, r)
        return Z, O

    def atencao(self, QKV, Bt, T, H):
        self.reg.confere_bloco("qkv", QKV)
        m, E = QKV
        D = m.shape[1] // 3
        self._formas_atencao("atencao", m, Bt, T, H, D)
        oacc = torch.empty(Bt * T, D, dtype=torch.int32, device=m.device)
        oe = torch.empty(Bt * T, D, dtype=torch.int16, device=m.device)
        P = torch.empty(Bt * H, T, T, dtype=torch.uint8, device=m.device)
        if ATENCAO_WS:
            nws = self.lib.jt_atencao_ws_bytes(Bt, T, H, D)
            ws = torch.empty(max(nws, 16), dtype=torch.uint8, device=m.device)
            self._lanca("atencao", "jt_atencao_ws", (m, E, oacc, oe, P, Bt, T, H, D, GA, ws, nws), dict(qkv=m, qkvE=E), (Bt * T, D),
                        longos=(11,))
        else:
            self._lanca("atencao", "jt_atencao", (m, E, oacc, oe, P, Bt, T, H, D, GA), dict(qkv=m, qkvE=E), (Bt * T, D))
        return (oacc, oe), P

    # no reference counterpart: attention whose outputs come already quantized (quant(atencao(...)) in one launch
    # sequence); where the kernels cannot (not head width 64 at BLK = 32), the op-by-op composition runs instead
    def _q_suportado(self, T, H, D):
        return ATENCAO_WS and BLK == 32 and H and D % H == 0 and D // H == 64 and T <= 512

    def atencao_q(self, QKV, Bt, T, H):
        """(quant(O), P) for (O, P) = atencao(QKV, Bt, T, H)."""
        m, E = QKV
        D = m.shape[1] // 3
        if not self._q_suportado(T, H, D):
            oc, P = self.atencao(QKV, Bt, T, H)
            return self.quant(oc), P
        self.reg.confere_bloco("qkv", QKV)
        self._formas_atencao("atencao", m, Bt, T, H, D)
        Om = self._novo_bloco(Bt * T, D, m.device)
        P = torch.empty(Bt * H, T, T, dtype=torch.uint8, device=m.device)
        nws = self.lib.jt_atencao_ws_bytes(Bt, T, H, D)
        ws = torch.empty(max(nws, 16), dtype=torch.uint8, device=m.device)
        self._lanca("atencao+quant", "jt_atencao_ws_q", (m, E, Om[0], Om[1], P, Bt, T, H, D, GA, ws, nws), dict(qkv=m, qkvE=E), (Bt * T, D),
                    longos=(11,))
        return Om, P

    def atencao_back_q(self, GO, QKV, P, Bt, T, H):
        """quant(atencao_back(GO, QKV, P, Bt, T, H))."""
        (gm, gE), (m, E) = GO, QKV
        D = gm.shape[1]
        if not self._q_suportado(T, H, D):
            return self.quant(self.atencao_back(GO, QKV, P, Bt, T, H))
        self.reg.confere_bloco("go", GO); self.reg.confere_bloco("qkv", QKV)
        self._formas_atencao("atencao_back", m, Bt, T, H, D)
        self.reg.exige(tuple(P.shape) == (Bt * H, T, T) and P.dtype == torch.uint8 and P.is_contiguous(),
                       f"atencao_back: P com forma {tuple(P.shape)}, esperado {(Bt * H, T, T)} uint8")
        G = self._novo_bloco(Bt * T, 3 * D, m.device)
        nws = self.lib.jt_atencao_back_ws_bytes(Bt, T, H, D)
        ws = torch.empty(max(nws, 16), dtype=torch.uint8, device=m.device)
        self._lanca("atencao_back+quant", "jt_atencao_back_ws_q", (gm, gE, m, E, P, G[0], G[1], Bt, T, H, D, GA, int(ATENCAO_LIMITE), ws, nws),
                    dict(go=gm, goE=gE, qkv=m, qkvE=E, P=P), (Bt * T, 3 * D), longos=(14,))
        return G

    # no reference counterpart: atencao_q / atencao_back_q converting q, k, v once for both. atencao_qs also returns a
    # buffer with the backward's conversions of q, k, v (None where the kernels do not run: then atencao_back_qs is
    # atencao_back_q); atencao_back_qs(GO, QKV, P, salvo, ...) reads them, for the same QKV, unchanged in between.
    def atencao_qs(self, QKV, Bt, T, H):
        """(quant(O), P, salvo) for (O, P) = atencao(QKV, Bt, T, H)."""
        m, E = QKV
        D = m.shape[1] // 3
        if not self._q_suportado(T, H, D):
            Om, P = self.atencao_q(QKV, Bt, T, H)
            return Om, P, None
        self.reg.confere_bloco("qkv", QKV)
        self._formas_atencao("atencao", m, Bt, T, H, D)
        Om = self._novo_bloco(Bt * T, D, m.device)
        P = torch.empty(Bt * H, T, T, dtype=torch.uint8, device=m.device)
        nws, ns = self.lib.jt_atencao_ws_bytes(Bt, T, H, D), self.lib.jt_atencao_salvo_bytes(Bt, T, H, D)
        ws = torch.empty(max(nws, 16), dtype=torch.uint8, device=m.device)
        salvo = torch.empty(max(ns, 16), dtype=torch.uint8, device=m.device)
        self._lanca("atencao+quant", "jt_atencao_ws_qs", (m, E, Om[0], Om[1], P, Bt, T, H, D, GA, ws, nws, salvo, ns), dict(qkv=m, qkvE=E),
                    (Bt * T, D), longos=(11, 13))
        return Om, P, salvo

    def atencao_back_qs(self, GO, QKV, P, salvo, Bt, T, H):
        """quant(atencao_back(GO, QKV, P, Bt, T, H)), with q, k, v converted by atencao_qs into salvo."""
        if salvo is None:
            return self.atencao_back_q(GO, QKV, P, Bt, T, H)
        (gm, gE), (m, E) = GO, QKV
        D = gm.shape[1]
        self.reg.confere_bloco("go", GO); self.reg.confere_bloco("qkv", QKV)
        self._formas_atencao("atencao_back", m, Bt, T, H, D)
        self.reg.exige(tuple(P.shape) == (Bt * H, T, T) and P.dtype == torch.uint8 and P.is_contiguous(),
                       f"atencao_back: P com forma {tuple(P.shape)}, esperado {(Bt * H, T, T)} uint8")
        ns = self.lib.jt_atencao_salvo_bytes(Bt, T, H, D)
        self.reg.exige(salvo.dtype == torch.uint8 and salvo.numel() >= ns, f"atencao_back: salvo com {salvo.numel()} bytes, esperado {ns}")
        G = self._novo_bloco(Bt * T, 3 * D, m.device)
        nws = self.lib.jt_atencao_back_ws_bytes(Bt, T, H, D)
        ws = torch.empty(max(nws, 16), dtype=torch.uint8, device=m.device)
        self._lanca("atencao_back+quant", "jt_atencao_back_ws_qs",
                    (gm, gE, m, E, P, G[0], G[1], Bt, T, H, D, GA, int(ATENCAO_LIMITE), ws, nws, salvo, ns),
                    dict(go=gm, goE=gE, qkv=m, qkvE=E, P=P), (Bt * T, 3 * D), longos=(14, 16))
        return G

    def _formas_atencao(self, op, m, Bt, T, H, D):
        """Head width hd = D/H: 4 is the spec's shape (ops.py:475: T a multiple of 32, H <= 64; here T up to 256);
        16, 32 and 64 run the generalized kernels (T a multiple of 64 up to 512)."""
        hd = D // H if H and D % H == 0 else 0
        if hd == 4:
            ok = T % 32 == 0 and 0 < T <= 256 and H <= 64
        else:
            ok = hd in (16, 32, 64) and T % 64 == 0 and 0 < T <= 512
        self.reg.exige(ok and m.shape[0] == Bt * T and m.shape[1] == 3 * D,
                       f"{op}: T={T}, D={D}, H={H} (cabeca 4: T multiplo de 32 ate 256 e H <= 64; cabeca 16, 32 ou 64: "
                       f"T multiplo de 64 ate 512)")

    def atencao_back(self, GO, QKV, P, Bt, T, H):
        self.reg.confere_bloco("go", GO); self.reg.confere_bloco("qkv", QKV)
        (gm, gE), (m, E) = GO, QKV
        D = gm.shape[1]
        self._formas_atencao("atencao_back", m, Bt, T, H, D)
        self.reg.exige(tuple(P.shape) == (Bt * H, T, T) and P.dtype == torch.uint8 and P.is_contiguous(),
                       f"atencao_back: P com forma {tuple(P.shape)}, esperado {(Bt * H, T, T)} uint8")
        acc = torch.empty(Bt * T, 3 * D, dtype=torch.int32, device=m.device)
        e = torch.empty(Bt * T, 3 * D, dtype=torch.int16, device=m.device)
        if ATENCAO_WS:
            nws = self.lib.jt_atencao_back_ws_bytes(Bt, T, H, D)
            ws = torch.empty(max(nws, 16), dtype=torch.uint8, device=m.device)
            self._lanca("atencao_back", "jt_atencao_back_ws", (gm, gE, m, E, P, acc, e, Bt, T, H, D, GA, int(ATENCAO_LIMITE), ws, nws),
                        dict(go=gm, goE=gE, qkv=m, qkvE=E, P=P), (Bt * T, 3 * D), longos=(14,))
        else:
            self._lanca("atencao_back", "jt_atencao_back", (gm, gE, m, E, P, acc, e, Bt, T, H, D, GA, int(ATENCAO_LIMITE)),
                        dict(go=gm, goE=gE, qkv=m, qkvE=E, P=P), (Bt * T, 3 * D))
        return acc, e

    def softmax_ce(self, L, alvo):
        self.reg.confere_cru("logits", L)
        acc, e = L
        M, V = acc.shape
        self.reg.exige(V <= 1024 and V % 128 == 0, f"softmax_ce: V={V}")
        g = self._novo_bloco(M, V, acc.device)
        d = torch.empty(M, dtype=torch.int32, device=acc.device)
        s = torch.empty(M, dtype=torch.int32, device=acc.device)
        self._lanca("softmax_ce", "jt_softmax_ce", (acc, e, alvo, g[0], g[1], d, s, M, V, int(math.log2(M))),
                    dict(acc=acc, e=e, alvo=alvo), (M, V))
        return g, d, s

    # no reference counterpart: the loss of modelo.py:93 from softmax_ce's rows in one launch
    def perda(self, d_alvo, soma):
        """mean(d_alvo / 256 + ln(soma / 4096)) in float64, a 0-dim tensor on the device."""
        M = d_alvo.shape[0] if d_alvo.dim() == 1 else -1
        self.reg.exige(d_alvo.dtype == torch.int32 and soma.dtype == torch.int32 and d_alvo.dim() == 1 and soma.shape == d_alvo.shape
                       and M > 0 and d_alvo.is_contiguous() and soma.is_contiguous(), "perda: d_alvo e soma int32 [M] contiguos")
        out = torch.empty((), dtype=torch.float64, device=d_alvo.device)
        self._lanca("perda", "jt_perda", (d_alvo, soma, out, M), dict(d_alvo=d_alvo, soma=soma), (M,))
        return out

    # ---------------------------------------------------------------- optimizer, in place (ops.py:504-515)
    def momento(self, Gc, Mom):
        self.reg.confere_cru("grad", Gc); self.reg.confere_bloco("momento", Mom)
        n = Mom[0].numel() // BLK
        self._lanca("momento", "jt_momento", (Gc[0], Gc[1], Mom[0], Mom[1], n), dict(g=Gc[0], ge=Gc[1]), tuple(Mom[0].shape), longos=(4,))
        return Mom

    # no reference counterpart: momento + peso of every tensor in one launch
    def tabela_otimizador(self, itens):
        """Device table for `otimizador`. itens: [(grad raw, Mom, W, R)] or [(grad raw, Mom, W, R, Wt)] with fixed
        addresses (updated in place); Wt = (mantissas [N, M], exponents [N, M / BLK]) receives transpoe(W) of the new
        weight (BLK 32, M % 32 == 0, N % 128 == 0 for every tensor of the table; None: not written). A gradient whose
        exponent tensor is a vector of M + N (gemm_cru_lote's compact form) is read as such."""
        itens = [tuple(it) + (None,) * (5 - len(it)) for it in itens]
        linhas, inicio, transpostas = [], 0, False
        for Gc, Mom, W, R, Wt in itens:
            M, N = W[0].shape
            compacto = Gc[1].dim() == 1 and Gc[0].dim() == 2
            if compacto:
                self.reg.exige(Gc[0].dtype == torch.int32 and Gc[1].dtype == torch.int16 and Gc[1].numel() == M + N and Gc[0].is_cuda
                               and Gc[0].is_contiguous() and Gc[1].is_contiguous() and N % 16 == 0,
                               f"otimizador: gradiente compacto (int32 {(M, N)}, int16 {(M + N,)}) esperado")
            else:
                self.reg.confere_cru("grad", Gc)
            for n, t in (("momento", Mom), ("W", W), ("residuo", R)):
                self.reg.confere_bloco(n, t)
            if Wt is not None:
                transpostas = True
                self.reg.confere_bloco("W transposta", Wt)
                self.reg.exige(tuple(Wt[0].shape) == (N, M), f"otimizador: transposta {tuple(Wt[0].shape)}, esperado {(N, M)}")
            nb = W[0].numel() // BLK
            self.reg.exige(Gc[0].numel() == W[0].numel() == Mom[0].numel() == R[0].numel(), "otimizador: formas diferentes")
            ptrs = [t.data_ptr() for t in (Gc[0], Gc[1], Mom[0], Mom[1], W[0], W[1], R[0], R[1])]
            ptrs += [Wt[0].data_ptr(), Wt[1].data_ptr()] if Wt is not None else [0, 0]
            linhas.append(ptrs + [inicio, nb, (N << 32) | M, int(compacto)])
            inicio += nb
        self.reg.exige(0 < len(linhas) <= 256, "otimizador: de 1 a 256 tensores")
        self.reg.exige(self.lib.jt_tab_otim_bytes() == 112, "otimizador: tamanho de entrada da tabela inesperado")
        if transpostas:
            self.reg.exige(BLK == 32 and all(W[0].shape[0] % 32 == 0 and W[0].shape[1] % 128 == 0 for _, _, W, _, _ in itens),
                           "otimizador com transpostas: BLK 32 e tensores com M % 32 == 0, N % 128 == 0")
        tab = torch.tensor(linhas, dtype=torch.int64).to(itens[0][2][0].device)
        # the table keeps every tensor whose address it holds alive for as long as it exists
        vivos = tuple(t for it in itens for x in it if x is not None for t in x)
        return tab, len(linhas), inicio, vivos, transpostas

    def otimizador(self, tabela, k, ef):
        """momento + peso of every tensor of the table (and the transposes of the new weights where it holds them)."""
        tab, ntab, nblocos = tabela[:3]
        fn = "jt_otimizador_t" if len(tabela) > 4 and tabela[4] else "jt_otimizador"
        self._lanca("otimizador", fn, (tab, ntab, nblocos, k, int(ef)), dict(), (nblocos * BLK,), longos=(2,))

    def peso(self, W, Mom, R, k, ef):
        for n, t in (("W", W), ("momento", Mom), ("residuo", R)):
            self.reg.confere_bloco(n, t)
        n = W[0].numel() // BLK
        self._lanca("peso", "jt_peso", (W[0], W[1], Mom[0], Mom[1], R[0], R[1], k, int(ef), n), dict(), tuple(W[0].shape), longos=(8,))
        return W, R
