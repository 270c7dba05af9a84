"""Argument guards of the attention entry points through the C ABI: GA, the guard bits of the aligned values
(ops.py:20 fixes it at 4), is taken from 0 to 4, the range every bound of the kernels assumes (aligned values of at
most 127 << 4 = 2032); any other value returns hipErrorInvalidValue before anything is launched, at head width 4
and 64, forward and backward, with and without a workspace."""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu
HIP_ERROR_INVALID_VALUE = 1


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


@pytest.mark.parametrize("GA", [-1, 5, 16])
@pytest.mark.parametrize("H", [64, 4])                         # head width 4 and 64 at D = 256, T = 128
def test_atencao_recusa_ga_fora(GA, H):
    """Every buffer has its real size for the shape (a guard that failed would launch on valid memory, not past a
    short buffer), and the outputs must keep the value they were filled with."""
    from jatai_amd import ops as O
    lib = O.carrega_lib()
    for f in ("jt_atencao", "jt_atencao_back", "jt_atencao_ws", "jt_atencao_back_ws", "jt_atencao_back_sem_alocar"):
        getattr(lib, f).restype = ctypes.c_int
    lib.jt_atencao_ws_bytes.restype = ctypes.c_longlong
    lib.jt_atencao_back_ws_bytes.restype = ctypes.c_longlong
    lib.jt_atencao_mfma(1)
    blk = O.BLK
    assert lib.jt_bloco(blk) == 0
    Bt, T, D = 1, 128, 256
    M = Bt * T
    z = lambda *forma, dt=torch.int8: torch.zeros(*forma, dtype=dt, device="cuda")
    s7 = lambda *forma, dt=torch.int8: torch.full(forma, 7, dtype=dt, device="cuda")
    qm, qE, gm, gE = z(M, 3 * D), z(M, 3 * D // blk), z(M, D), z(M, D // blk)
    P = z(Bt * H, T, T, dt=torch.uint8)
    oacc, oe, Pout = s7(M, D, dt=torch.int32), s7(M, D, dt=torch.int16), s7(Bt * H, T, T, dt=torch.uint8)
    gacc, ge = s7(M, 3 * D, dt=torch.int32), s7(M, 3 * D, dt=torch.int16)
    wf = s7(max(64, lib.jt_atencao_ws_bytes(Bt, T, H, D)), dt=torch.uint8)
    wb = s7(max(64, lib.jt_atencao_back_ws_bytes(Bt, T, H, D)), dt=torch.uint8)
    p = _p
    assert lib.jt_atencao(p(qm), p(qE), p(oacc), p(oe), p(Pout), Bt, T, H, D, GA, 0) == HIP_ERROR_INVALID_VALUE
    assert lib.jt_atencao_back(p(gm), p(gE), p(qm), p(qE), p(P), p(gacc), p(ge), Bt, T, H, D, GA, 0, 0) == HIP_ERROR_INVALID_VALUE
    assert lib.jt_atencao_ws(p(qm), p(qE), p(oacc), p(oe), p(Pout), Bt, T, H, D, GA, p(wf), ctypes.c_longlong(wf.numel()),
                             0) == HIP_ERROR_INVALID_VALUE
    assert lib.jt_atencao_back_ws(p(gm), p(gE), p(qm), p(qE), p(P), p(gacc), p(ge), Bt, T, H, D, GA, 0, p(wb),
                                  ctypes.c_longlong(wb.numel()), 0) == HIP_ERROR_INVALID_VALUE
    assert lib.jt_atencao_back_sem_alocar(p(gm), p(gE), p(qm), p(qE), p(P), p(gacc), p(ge), Bt, T, H, D, GA, 0,
                                          0) == HIP_ERROR_INVALID_VALUE
    torch.cuda.synchronize()
    for nome, t in (("oacc", oacc), ("oe", oe), ("P", Pout), ("gacc", gacc), ("ge", ge), ("ws", wf), ("ws back", wb)):
        assert bool((t == 7).all()), nome


def test_otimizador_t_e_janelas_recusam():
    """jt_otimizador_t refuses BLK 128, a block count that is not a whole number of 32 x 128 tiles and a table of 0
    or more than 256 entries (a count of 0 is a no-op); jt_janelas refuses a corpus shorter than one window and
    misaligned start or token buffers. The table is a real one and every buffer is larger than the shape asks, so
    a guard that failed would launch on valid memory; the outputs must keep their values."""
    from jatai_amd import ops as O
    from jatai_amd.registro import Registro
    lib = O.carrega_lib()
    for f in ("jt_otimizador_t", "jt_janelas", "jt_bloco"):
        getattr(lib, f).restype = ctypes.c_int
    blk0 = O.BLK
    try:
        O.BLK = 32
        ops = O.OpsHip(Registro("/tmp/jt_guardas", "g", eco=False))
        assert lib.jt_bloco(32) == 0
        M, N = 32, 128
        g = torch.Generator().manual_seed(3)
        W = (torch.randint(-100, 100, (M, N), generator=g, dtype=torch.int8).cuda(), torch.zeros(M, N // 32, dtype=torch.int8, device="cuda"))
        Mom = (torch.zeros(M, N, dtype=torch.int8, device="cuda"), torch.full((M, N // 32), O.E_ZERO, dtype=torch.int8, device="cuda"))
        R = (torch.zeros(M, N, dtype=torch.int8, device="cuda"), torch.full((M, N // 32), O.E_ZERO, dtype=torch.int8, device="cuda"))
        G = (torch.randint(-1000, 1000, (M, N), generator=g, dtype=torch.int32).cuda(), torch.full((M, N), -20, dtype=torch.int16, device="cuda"))
        Wt = (torch.full((N, M), 7, dtype=torch.int8, device="cuda"), torch.full((N, M // 32), 7, dtype=torch.int8, device="cuda"))
        tab, ntab, nb, vivos, tr = ops.tabela_otimizador([(G, Mom, W, R, Wt)])
        assert ntab == 1 and nb == 128 and tr
        w0 = W[0].clone()
        p = ctypes.c_void_p(tab.data_ptr())
        ll = ctypes.c_longlong
        assert lib.jt_otimizador_t(p, 1, ll(0), 4, 1, 0) == 0                      # nothing to do
        assert lib.jt_otimizador_t(p, 1, ll(129), 4, 1, 0) == HIP_ERROR_INVALID_VALUE
        assert lib.jt_otimizador_t(p, 0, ll(128), 4, 1, 0) == HIP_ERROR_INVALID_VALUE
        assert lib.jt_otimizador_t(p, 257, ll(128), 4, 1, 0) == HIP_ERROR_INVALID_VALUE
        assert lib.jt_bloco(128) == 0
        assert lib.jt_otimizador_t(p, 1, ll(128), 4, 1, 0) == HIP_ERROR_INVALID_VALUE
        assert lib.jt_bloco(32) == 0
        torch.cuda.synchronize()
        assert torch.equal(W[0], w0) and bool((Wt[0] == 7).all()) and bool((Wt[1] == 7).all())
        # windows: a 4096-byte corpus buffer, told n = T (one byte short of a window)
        T, Bt = 64, 2
        corpus = torch.randint(0, 256, (4096,), generator=g, dtype=torch.uint8).cuda()
        ini = torch.zeros(4, dtype=torch.int64, device="cuda")
        tok = torch.full((4 * Bt * T,), 7, dtype=torch.int32, device="cuda")
        alvo = torch.full_like(tok, 7)
        c, i, t, a = (ctypes.c_void_p(x.data_ptr()) for x in (corpus, ini, tok, alvo))
        desl = lambda x, b: ctypes.c_void_p(x.data_ptr() + b)
        assert lib.jt_janelas(c, ll(T), i, t, a, Bt, T, 0) == HIP_ERROR_INVALID_VALUE
        assert lib.jt_janelas(c, ll(4096), desl(ini, 4), t, a, Bt, T, 0) == HIP_ERROR_INVALID_VALUE
        assert lib.jt_janelas(c, ll(4096), i, desl(tok, 2), a, Bt, T, 0) == HIP_ERROR_INVALID_VALUE
        assert lib.jt_janelas(c, ll(4096), i, t, desl(alvo, 2), Bt, T, 0) == HIP_ERROR_INVALID_VALUE
        assert lib.jt_janelas(c, ll(4096), i, t, a, 0, T, 0) == HIP_ERROR_INVALID_VALUE
        torch.cuda.synchronize()
        assert bool((tok == 7).all()) and bool((alvo == 7).all())
        assert lib.jt_janelas(c, ll(4096), i, t, a, Bt, T, 0) == 0                  # the same call, well formed
        torch.cuda.synchronize()
        assert torch.equal(tok[:T].cpu(), corpus[:T].cpu().int()) and torch.equal(alvo[:T].cpu(), corpus[1:T + 1].cpu().int())
    finally:
        O.BLK = blk0
        lib.jt_bloco(blk0)
