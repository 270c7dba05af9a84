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
    from jatai_amd import ops as O
    lib = O.carrega_lib()
    for f in ("jt_atencao", "jt_atencao_back", "jt_atencao_ws", "jt_atencao_back_ws", "jt_atencao_back_sem_alocar"):
        getattr(lib, f).restype = ctypes.c_int
    Bt, T, D = 1, 128, 256
    t = torch.zeros(16, dtype=torch.int8, device="cuda")
    sentinela = torch.full((64,), 7, dtype=torch.int8, device="cuda")   # would be overwritten by any launch
    p, s = _p(t), _p(sentinela)
    assert lib.jt_atencao(p, p, s, s, s, Bt, T, H, D, GA, 0) == HIP_ERROR_INVALID_VALUE
    assert lib.jt_atencao_back(p, p, p, p, p, s, s, Bt, T, H, D, GA, 0, 0) == HIP_ERROR_INVALID_VALUE
    assert lib.jt_atencao_ws(p, p, s, s, s, Bt, T, H, D, GA, s, ctypes.c_longlong(64), 0) == HIP_ERROR_INVALID_VALUE
    assert lib.jt_atencao_back_ws(p, p, p, p, p, s, s, Bt, T, H, D, GA, 0, s, ctypes.c_longlong(64), 0) == HIP_ERROR_INVALID_VALUE
    assert lib.jt_atencao_back_sem_alocar(p, p, p, p, p, s, s, Bt, T, H, D, GA, 0, 0) == HIP_ERROR_INVALID_VALUE
    torch.cuda.synchronize()
    assert bool((sentinela == 7).all())
