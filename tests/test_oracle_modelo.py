"""The CPU oracle composed as the full training step (jatai_amd.modelo.Modelo with OpsOraculo) reproduces every
op output of the spec's first two training steps (tests/golden/trace_r.json, modelo.py:51-140 with OpsRef)."""
import traco as TR
from backends import host
from oracle.ops_oracle import OpsOraculo


def test_oraculo_dois_passos_vs_spec():
    _, init, passos = TR.roda(OpsOraculo(128), TR.RegStub(), "cpu", 2, host)
    TR.confere(init, passos)
