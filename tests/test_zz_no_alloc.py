"""jt_atencao_back_sem_alocar (the attention backward with its workspace in the library's fixed device array
`scratch`, for callers that cannot allocate) through the C ABI: its raw gradient equals jt_atencao_back_ws's with a
caller workspace, bit for bit, on two calls in a row -- the second with a smaller input, so that the array holds
the first call's contents when the second starts -- in both backward variants. A shape whose workspace exceeds the
array is refused with hipErrorOutOfMemory and launches nothing."""
import ctypes

import pytest
import torch

import recipe as R
from backends import host, primeira_diferenca

pytestmark = pytest.mark.gpu
HIP_ERROR_OUT_OF_MEMORY = 2


def _lib():
    from jatai_amd import ops as O
    lib = O.carrega_lib()
    lib.jt_atencao_back_sem_alocar.restype = ctypes.c_int
    lib.jt_atencao_back_ws.restype = ctypes.c_int
    lib.jt_scratch_bytes.restype = ctypes.c_longlong
    lib.jt_atencao_back_ws_bytes.restype = ctypes.c_longlong
    lib.jt_atencao.restype = ctypes.c_int
    return lib


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _entradas(seed, Bt, T, H, D, blk=32):
    M = Bt * T
    dev = lambda a: torch.from_numpy(a).cuda()
    q = tuple(dev(v) for v in R.bloco(R.substream(seed, "qkv"), M, 3 * D, blk, espalha=4, e0=-7, zera=0.05))
    g = tuple(dev(v) for v in R.bloco(R.substream(seed, "go"), M, D, blk, espalha=4, e0=-20, zera=0.05))
    return q, g


def _chama(lib, fn, q, g, P, Bt, T, H, D, limite, ws=None):
    M = Bt * T
    acc = torch.full((M, 3 * D), 7, dtype=torch.int32, device="cuda")
    e = torch.full((M, 3 * D), 7, dtype=torch.int16, device="cuda")
    args = [_p(g[0]), _p(g[1]), _p(q[0]), _p(q[1]), _p(P), _p(acc), _p(e), Bt, T, H, D, 4, int(limite)]
    if ws is not None:
        args += [_p(ws), ctypes.c_longlong(ws.numel())]
    rc = getattr(lib, fn)(*args, 0)
    torch.cuda.synchronize()
    return rc, acc, e


@pytest.mark.parametrize("limite", [False, True])
def test_sem_alocar_igual_ao_workspace(limite):
    lib = _lib()
    assert lib.jt_bloco(32) == 0
    D, H = 512, 8
    for Bt, T in ((8, 256), (2, 128)):              # the second call smaller than the first
        print(f"sem_alocar: Bt={Bt} T={T} limite={limite}", flush=True)
        assert lib.jt_atencao_back_ws_bytes(Bt, T, H, D) <= lib.jt_scratch_bytes()
        q, g = _entradas(R.substream(808, f"{Bt} {T}"), Bt, T, H, D)
        oacc = torch.empty(Bt * T, D, dtype=torch.int32, device="cuda")
        oe = torch.empty(Bt * T, D, dtype=torch.int16, device="cuda")
        P = torch.empty(Bt * H, T, T, dtype=torch.uint8, device="cuda")
        assert lib.jt_atencao(_p(q[0]), _p(q[1]), _p(oacc), _p(oe), _p(P), Bt, T, H, D, 4, 0) == 0
        ws = torch.empty(lib.jt_atencao_back_ws_bytes(Bt, T, H, D), dtype=torch.uint8, device="cuda")
        rc1, a1, e1 = _chama(lib, "jt_atencao_back_ws", q, g, P, Bt, T, H, D, limite, ws)
        rc2, a2, e2 = _chama(lib, "jt_atencao_back_sem_alocar", q, g, P, Bt, T, H, D, limite)
        assert rc1 == 0 and rc2 == 0, (rc1, rc2)
        for nome, x, y in (("acc", a2, a1), ("e", e2, e1)):
            d = primeira_diferenca(host(x), host(y))
            assert d is None, f"Bt={Bt} T={T} {nome}: (flat index, fixed scratch, workspace, count) = {d}"


def test_sem_alocar_recusa_acima_do_maximo():
    """Every buffer at its real size for the shape (so a broken guard could not touch memory it does not own), the
    matrix-core family selected (the path that reaches the size check), and the outputs left as filled."""
    lib = _lib()
    assert lib.jt_bloco(32) == 0
    lib.jt_atencao_mfma(1)
    Bt, T, H, D = 64, 256, 8, 512                    # config 5: about 200 MB of workspace
    M = Bt * T
    assert lib.jt_atencao_back_ws_bytes(Bt, T, H, D) > lib.jt_scratch_bytes()
    q, g = _entradas(R.substream(809, "recusa"), Bt, T, H, D)
    P = torch.zeros(Bt * H, T, T, dtype=torch.uint8, device="cuda")
    acc = torch.full((M, 3 * D), 7, dtype=torch.int32, device="cuda")
    e = torch.full((M, 3 * D), 7, dtype=torch.int16, device="cuda")
    rc = lib.jt_atencao_back_sem_alocar(_p(g[0]), _p(g[1]), _p(q[0]), _p(q[1]), _p(P), _p(acc), _p(e), Bt, T, H, D, 4, 0, 0)
    torch.cuda.synchronize()
    assert rc == HIP_ERROR_OUT_OF_MEMORY
    assert bool((acc == 7).all()) and bool((e == 7).all())
