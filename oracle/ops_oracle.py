"""`OpsOraculo`: the CPU oracle behind the reference operator surface -- TEST INFRASTRUCTURE ONLY.

Same methods, arguments and return structure as the reference spec `OpsRef` (jatai_cuda/ops.py:92-290) and
the reference wrapper `OpsCuda` (ops.py:294-515, including the R16 trio para16/para8/soma16), computed by
`libjatai_oracle.so` (int64 C++ restatement, jatai_oracle.cpp) on CPU torch tensors. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module.

Block size and the attention-backward variant are attributes (`blk`, `limite`) instead of module globals.
"""
import ctypes
import math
import os

import numpy as np
import torch

AQUI = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(AQUI, "libjatai_oracle.so")
E_ZERO = -127
GA = 4

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            raise RuntimeError(f"oracle library missing: build it with `make -C {AQUI}`")
        _lib = ctypes.CDLL(LIB)
        for f in ("or_embed", "or_um_quente", "or_softmax_ce"):
            getattr(_lib, f).restype = ctypes.c_int
    return _lib


def _p(t):
    assert t.device.type == "cpu" and t.is_contiguous(), "oracle takes contiguous CPU tensors"
    return ctypes.c_void_p(t.data_ptr())


def _ll(x):
    return ctypes.c_longlong(int(x))


def _i(x):
    return ctypes.c_int(int(x))


def _cpu(t):
    return t.detach().to("cpu").contiguous()


def g_rms(D, blk):
    G, GB = ctypes.c_int(), ctypes.c_int()
    lib().or_g_rms(_i(D), _i(blk), ctypes.byref(G), ctypes.byref(GB))
    return G.value, GB.value


class OpsOraculo:
    nome = "oraculo"

    def __init__(self, blk=128, limite=False, estocastico=False):
        # estocastico: gemm_soma's residual add rounds stochastically, as OpsCuda with jt_res_estocastico(1)
        self.blk, self.limite, self.estocastico = blk, limite, estocastico

    def _bloco(self, R, C, dt=torch.int8):
        return torch.empty(R, C, dtype=dt), torch.empty(R, C // self.blk, dtype=torch.int8)

    # ---- primitives
    @staticmethod
    def prim(nome, *arrs):
        arrs = [np.ascontiguousarray(a, dtype=np.int64) for a in arrs]
        out = np.empty_like(arrs[0])
        getattr(lib(), "or_" + nome)(*[a.ctypes.data_as(ctypes.c_void_p) for a in arrs],
                                     out.ctypes.data_as(ctypes.c_void_p), _ll(out.size))
        return out

    # ---- GEMM family (ops.py:95-119)
    def gemm(self, A, B, cru=False):
        (a, ea), (b, eb) = [tuple(_cpu(t) for t in X) for X in (A, B)]
        M, K = a.shape
        N = b.shape[0]
        if cru:
            C = (torch.empty(M, N, dtype=torch.int32), torch.empty(M, N, dtype=torch.int16))
            lib().or_gemm(_p(a), _p(ea), _p(b), _p(eb), _i(M), _i(N), _i(K), _i(self.blk), _i(1), None, None, _p(C[0]), _p(C[1]))
        else:
            C = self._bloco(M, N)
            lib().or_gemm(_p(a), _p(ea), _p(b), _p(eb), _i(M), _i(N), _i(K), _i(self.blk), _i(0), _p(C[0]), _p(C[1]), None, None)
        return C

    def gemm_soma(self, A, B, X):
        return (self.soma_est if self.estocastico else self.soma)(X, self.gemm(A, B))

    def soma_est(self, X, Y):
        """soma(X, Y) with gemm_soma's stochastic residual rounding (jatai_cuda.cu:146-159, :375); the seeds follow
        the positions of Y's values in its [R, C] matrix."""
        (xm, xE), (ym, yE) = [tuple(_cpu(t) for t in T) for T in (X, Y)]
        R, C = xm.shape
        Z = self._bloco(R, C)
        lib().or_soma_est(_p(xm), _p(xE), _p(ym), _p(yE), _ll(R), _i(C), _i(self.blk), _p(Z[0]), _p(Z[1]))
        return Z

    def gemm_relu2(self, A, B):
        h = self.gemm(A, B)
        return h, self.relu2(h)

    def gemm_relu2_back(self, A, B, Hh):
        return self.relu2_back(self.gemm(A, B), Hh)

    def transpoe(self, X):
        m, E = (_cpu(t) for t in X)
        R, C = m.shape
        Y = self._bloco(C, R)
        lib().or_transpoe(_p(m), _p(E), _i(R), _i(C), _i(self.blk), _p(Y[0]), _p(Y[1]))
        return Y

    def de_f32(self, x):
        """float32 [R, C] to a block tensor: the exact split x = v 2^e (frexp, |v| < 2^24) as a raw int32 / int16
        tensor, then the spec's quant (ops.py:58-72)."""
        x = np.ascontiguousarray(_cpu(x).numpy().astype(np.float32))
        if not np.isfinite(x).all():
            raise ValueError("de_f32: non-finite input")
        m, e = np.frexp(x)
        v = (m.astype(np.float64) * float(1 << 24)).astype(np.int32)
        return self.quant((torch.from_numpy(v), torch.from_numpy((e - 24).astype(np.int16))))

    def quant(self, Cc):
        acc, e = (_cpu(t) for t in Cc)
        R, C = acc.shape
        Y = self._bloco(R, C)
        lib().or_quant(_p(acc), _p(e), _ll(R), _i(C), _i(self.blk), _p(Y[0]), _p(Y[1]))
        return Y

    def soma(self, X, Y):
        (xm, xE), (ym, yE) = [tuple(_cpu(t) for t in T) for T in (X, Y)]
        R, C = xm.shape
        Z = self._bloco(R, C)
        lib().or_soma(_p(xm), _p(xE), _p(ym), _p(yE), _ll(R), _i(C), _i(self.blk), _p(Z[0]), _p(Z[1]))
        return Z

    def relu2(self, Hh):
        m, E = (_cpu(t) for t in Hh)
        R, C = m.shape
        Z = self._bloco(R, C)
        lib().or_relu2(_p(m), _p(E), _ll(R), _i(C), _i(self.blk), _p(Z[0]), _p(Z[1]))
        return Z

    def relu2_back(self, Gg, Hh):
        (g, gE), (h, hE) = [tuple(_cpu(t) for t in T) for T in (Gg, Hh)]
        R, C = g.shape
        Z = self._bloco(R, C)
        lib().or_relu2_back(_p(g), _p(gE), _p(h), _p(hE), _ll(R), _i(C), _i(self.blk), _p(Z[0]), _p(Z[1]))
        return Z

    def embed(self, W, tok):
        m, E = (_cpu(t) for t in W)
        tok = _cpu(tok).to(torch.int32).contiguous()
        V, D = m.shape
        M = tok.numel()
        X = self._bloco(M, D)
        bad = lib().or_embed(_p(m), _p(E), _p(tok), _i(M), _i(D), _i(V), _i(self.blk), _p(X[0]), _p(X[1]))
        if bad:
            raise IndexError(f"embed: {bad} tokens outside the vocabulary of {V}")
        return X

    def um_quente(self, tok, V):
        tok = _cpu(tok).to(torch.int32).contiguous()
        M = tok.numel()
        U = self._bloco(M, V)
        bad = lib().or_um_quente(_p(tok), _i(M), _i(V), _i(self.blk), _p(U[0]), _p(U[1]))
        if bad:
            raise IndexError(f"um_quente: {bad} tokens outside the vocabulary of {V}")
        return U

    def rms(self, X):
        m, E = (_cpu(t) for t in X)
        M, D = m.shape
        Y = self._bloco(M, D)
        r, emax = torch.empty(M, dtype=torch.int32), torch.empty(M, dtype=torch.int32)
        lib().or_rms(_p(m), _p(E), _i(M), _i(D), _i(self.blk), _p(Y[0]), _p(Y[1]), _p(r), _p(emax))
        return Y, (r, emax)

    def rms_back(self, Gg, Y, cache):
        (g, gE), (y, yE) = [tuple(_cpu(t) for t in T) for T in (Gg, Y)]
        r, emax = _cpu(cache[0]), _cpu(cache[1])
        M, D = g.shape
        O = self._bloco(M, D)
        lib().or_rms_back(_p(g), _p(gE), _p(y), _p(yE), _p(r), _p(emax), _i(M), _i(D), _i(self.blk), _p(O[0]), _p(O[1]))
        return O

    def atencao(self, QKV, Bt, T, H):
        m, E = (_cpu(t) for t in QKV)
        D = m.shape[1] // 3
        oacc = torch.empty(Bt * T, D, dtype=torch.int32)
        oe = torch.empty(Bt * T, D, dtype=torch.int16)
        P = torch.empty(Bt * H, T, T, dtype=torch.uint8)
        lib().or_atencao(_p(m), _p(E), _i(Bt), _i(T), _i(H), _i(D), _i(self.blk), _i(GA), _p(oacc), _p(oe), _p(P))
        return (oacc, oe), P

    def atencao_back(self, GO, QKV, P, Bt, T, H):
        (gm, gE), (m, E) = [tuple(_cpu(t) for t in X) for X in (GO, QKV)]
        P = _cpu(P)
        D = gm.shape[1]
        acc = torch.empty(Bt * T, 3 * D, dtype=torch.int32)
        e = torch.empty(Bt * T, 3 * D, dtype=torch.int16)
        lib().or_atencao_back(_p(gm), _p(gE), _p(m), _p(E), _p(P), _i(Bt), _i(T), _i(H), _i(D), _i(self.blk), _i(GA),
                              _i(int(self.limite)), _p(acc), _p(e))
        return acc, e

    def softmax_ce(self, L, alvo):
        acc, e = (_cpu(t) for t in L)
        alvo = _cpu(alvo).to(torch.int32).contiguous()
        M, V = acc.shape
        g = self._bloco(M, V)
        d = torch.empty(M, dtype=torch.int32)
        s = torch.empty(M, dtype=torch.int32)
        bad = lib().or_softmax_ce(_p(acc), _p(e), _p(alvo), _i(M), _i(V), _i(self.blk), _p(g[0]), _p(g[1]), _p(d), _p(s))
        if bad:
            raise IndexError(f"softmax_ce: {bad} targets outside the vocabulary of {V}")
        return g, d, s

    def momento(self, Gc, Mom):
        g, ge = (_cpu(t) for t in Gc)
        mm, mE = Mom
        assert mm.device.type == "cpu" and mm.is_contiguous() and mE.is_contiguous()
        lib().or_momento(_p(g), _p(ge), _p(mm), _p(mE), _ll(mm.numel()), _i(self.blk))
        return Mom

    def peso(self, W, Mom, R, k, ef):
        (wm, wE), (rm, rE) = W, R
        mm, mE = (_cpu(t) for t in Mom)
        lib().or_peso(_p(wm), _p(wE), _p(mm), _p(mE), _p(rm), _p(rE), _i(k), _i(int(ef)), _ll(wm.numel()), _i(self.blk))
        return W, R

    # ---- 16-bit residual stream (jatai_cuda.cu:446-531; ops.py:406-426)
    def para16(self, X):
        m, E = (_cpu(t) for t in X)
        R, C = m.shape
        Z = self._bloco(R, C, torch.int16)
        lib().or_para16(_p(m), _p(E), _ll(m.numel()), _i(self.blk), _p(Z[0]), _p(Z[1]))
        return Z

    def para8(self, X16):
        m, E = (_cpu(t) for t in X16)
        R, C = m.shape
        Z = self._bloco(R, C)
        lib().or_para8(_p(m), _p(E), _ll(m.numel()), _i(self.blk), _p(Z[0]), _p(Z[1]))
        return Z

    def soma16(self, X16, Y):
        (xm, xE), (ym, yE) = [tuple(_cpu(t) for t in T) for T in (X16, Y)]
        R, C = xm.shape
        Z = self._bloco(R, C, torch.int16)
        lib().or_soma16(_p(xm), _p(xE), _p(ym), _p(yE), _ll(xm.numel()), _i(self.blk), _p(Z[0]), _p(Z[1]))
        return Z


def log2i(n):
    return int(math.log2(n))


def _plano(x):
    if torch.is_tensor(x):
        return [x]
    if isinstance(x, (tuple, list)):
        return [t for y in x for t in _plano(y)]
    return []


def _copia(x):
    if torch.is_tensor(x):
        return x.detach().cpu().clone()
    if isinstance(x, tuple):
        return tuple(_copia(y) for y in x)
    if isinstance(x, list):
        return [_copia(y) for y in x]
    return x


class OpsConferido:
    """The reference's checked wrapper (jatai_cuda/ops.py:519-560): every op runs on the backend under test
    (default: OpsHip, the HIP path) and on this oracle with the same inputs, and must agree bit for bit; the
    backend's outputs are returned. A mismatch fails through the Registro with the op, the output, the count of
    differing values and the first one, as ops.py:519-529 does. The oracle's inputs are copied before the
    backend runs (momento and peso update their arguments in place); block size and the attention variant follow
    jatai_amd.ops.BLK and ATENCAO_LIMITE at each call. A debugging aid: test infrastructure, like this module."""
    nome = "conferido"
    NOMES = {"rms": ["mantissa", "expoente", "r", "emax"], "atencao": ["o acc", "o exp", "P"],
             "softmax_ce": ["g mantissa", "g expoente", "d_alvo", "soma"], "peso": ["W", "W exp", "residuo", "residuo exp"],
             "gemm_relu2": ["h mantissa", "h expoente", "a mantissa", "a expoente"]}

    def __init__(self, reg, ops=None):
        from jatai_amd import ops as O
        self.O, self.reg = O, reg
        self.c = ops if ops is not None else O.OpsHip(reg)
        self.lib = getattr(self.c, "lib", None)
        self.n = {}

    def _compara(self, op, a, b, nome):
        a, b = a.detach().cpu(), b.detach().cpu()
        if tuple(a.shape) != tuple(b.shape):
            self.reg.falha(f"conferencia '{op}' / {nome}: forma HIP {tuple(a.shape)} x oraculo {tuple(b.shape)}")
        dif = a != b
        if not bool(dif.any()):
            return
        n = int(dif.sum())
        pos = dif.nonzero()[0].tolist()
        self.reg.falha(f"conferencia '{op}' / {nome}: {n} de {a.numel()} valores diferentes do oraculo.\n"
                       f"  primeiro em {pos}: HIP = {a[tuple(pos)].item()}, oraculo = {b[tuple(pos)].item()}", op=op, n_dif=n, pos=pos)

    def __getattr__(self, op):
        fc = getattr(self.c, op)
        if not callable(fc) or op.startswith("_"):
            return fc

        def f(*args, **kw):
            r = OpsOraculo(self.O.BLK, self.O.ATENCAO_LIMITE)
            fr = getattr(r, op)
            ra = _copia(args)
            out_c = fc(*args, **kw)
            out_r = fr(*ra, **{k: v for k, v in kw.items() if k == "cru"})
            nomes = self.NOMES.get(op, ["mantissa/acc", "expoente"])
            for i, (a, b) in enumerate(zip(_plano(out_c), _plano(out_r))):
                self._compara(op, a, b, nomes[i] if i < len(nomes) else f"saida {i}")
            self.n[op] = self.n.get(op, 0) + 1
            return out_c
        return f
