"""The C-ABI library loads (without touching a GPU) and exports every symbol include/jatai.h declares."""
import ctypes
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declarados():
    txt = open(os.path.join(ROOT, "include", "jatai.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(jt_\w+)\s*\(", txt)))


def test_exporta_tudo_do_cabecalho():
    import torch  # noqa: F401  (the library binds to the HIP runtime torch loads)
    from jatai_amd import ops as O
    lib = O.carrega_lib()
    nomes = _declarados()
    assert len(nomes) >= 29
    faltam = [n for n in nomes if not hasattr(lib, n)]
    assert not faltam, f"missing exports: {faltam}"


def test_superficie_python_usa_so_simbolos_declarados():
    from jatai_amd import ops as O
    assert set(O.FUNCOES) | set(O.VOIDS) <= set(_declarados())


def test_guardas_de_host_sem_gpu():
    """Format guards fire on the host before any launch (the reference's guards: jatai_cuda/registro.py:161-189)."""
    import pytest
    import torch
    from jatai_amd import ops as O
    from jatai_amd.registro import ErroJatai, Registro
    reg = Registro("/tmp/jatai_testes", "abi", eco=False)
    with pytest.raises(ErroJatai, match="not on the GPU"):
        reg.confere_bloco("A", (torch.zeros(4, 128, dtype=torch.int8), torch.zeros(4, 1, dtype=torch.int8)))
    O.BLK = 32
    try:
        with pytest.raises(ErroJatai, match="exponent shape"):
            reg.confere_bloco("A", (torch.zeros(4, 128, dtype=torch.int8), torch.zeros(4, 1, dtype=torch.int8)))
    finally:
        O.BLK = 128
    with pytest.raises(ErroJatai, match="int16"):
        reg.confere_cru("C", (torch.zeros(4, 128, dtype=torch.int32), torch.zeros(4, 128, dtype=torch.int32)))
