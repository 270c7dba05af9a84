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


def test_registro_estatistica_e_mensagens(tmp_path, capsys):
    """Host registry without a GPU: the block-tensor statistics (zero blocks, exponent range and median, mantissa
    bits of block maxima, zero and saturated mantissas) on a hand-built tensor, the warnings they trigger, and the
    error text (step and scope first, then the message) with its log record."""
    import json
    import pytest
    import torch
    from jatai_amd import ops as O
    from jatai_amd.registro import ErroJatai, Registro
    old = O.BLK
    O.BLK = 32
    try:
        reg = Registro(str(tmp_path), "r", eco=False)
        reg.novo_passo(3)
        m = torch.zeros(2, 64, dtype=torch.int8)
        m[0, :32] = torch.arange(-16, 16, dtype=torch.int8)          # block maximum 16: 5 bits; one zero
        m[1, 32:] = 127                                              # saturated block
        E = torch.tensor([[-115, -127], [-127, 3]], dtype=torch.int8)  # two zero blocks
        rec = reg.estatistica("x", (m, E))
        assert rec["blocos"] == 4 and rec["blocos_zero"] == 0.5
        assert (rec["exp_min"], rec["exp_max"]) == (-115, 3) and rec["bits_usados"] == 6.0
        assert rec["zeros_em_vivos"] == round(1 / 64, 4) and rec["saturados"] == 0.5
        err = capsys.readouterr().err
        assert "within 16 of the INT8 exponent range" in err and "mantissa bits" not in err
        z = reg.estatistica("z", (torch.zeros(1, 32, dtype=torch.int8), torch.full((1, 1), -127, dtype=torch.int8)))
        assert z["blocos_zero"] == 1.0 and "every block is zero" in capsys.readouterr().err
        with reg.trecho("forward"), reg.trecho("mlp"):
            with pytest.raises(ErroJatai) as e:
                reg.exige(False, "bad shape")
        assert str(e.value) == "step 3, forward / mlp:\nbad shape"
        linhas = [json.loads(l) for l in open(tmp_path / "r.jsonl")]
        assert [l["tipo"] for l in linhas].count("estatistica") == 2 and linhas[-1]["tipo"] == "erro"
        assert linhas[-1]["trecho"] == "forward / mlp" and linhas[-1]["passo"] == 3
    finally:
        O.BLK = old
