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
