"""The CPU oracle composed as the full training step (jatai_amd.modelo.Modelo with OpsOraculo) reproduces every
op output of the spec's first two training steps at the reference shape, at Bt = 8 and Bt = 16
(tests/golden/trace_r.json, trace_r_bt16.json: modelo.py:51-140 with OpsRef)."""
import pytest

import traco as TR
from backends import host
from oracle.ops_oracle import OpsOraculo


@pytest.mark.parametrize("nome", TR.TRACOS)
def test_oraculo_dois_passos_vs_spec(nome):
    _, init, passos = TR.roda(OpsOraculo(128), TR.RegStub(), "cpu", 2, host, nome)
    TR.confere(init, passos, nome)
