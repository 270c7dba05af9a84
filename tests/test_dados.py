"""The byte data path (jatai_amd/dados.py) against the reference's own `carregar` / `lote`
(treino_int8_gpu/treino.py:29-44), run on the synthetic UTF-8 corpus of tests/recipe.py by
tests/golden/make_dados.py (dados.json holds hashes, starts and leading bytes only), and against what the split
rule fixes line by line."""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

import recipe as R
from jatai_amd import dados as DD

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "dados.json")


def _sha(t):
    return hashlib.sha256(np.ascontiguousarray(t.cpu().numpy().astype(np.int64)).tobytes()).hexdigest()


@pytest.fixture(scope="module")
def corpus(tmp_path_factory):
    p = tmp_path_factory.mktemp("corpus")
    textos = R.corpus_sintetico(str(p))
    return str(p), textos


def test_carregar_vs_referencia(corpus):
    g = json.load(open(GOLD))["carregar"]
    tr, val = DD.carregar(corpus[0])
    for t, ref in ((tr, g["treino"]), (val, g["val"])):
        assert t.dtype == torch.int64 and len(t) == ref["n"] and t[:64].tolist() == ref["inicio"]
        assert _sha(t) == ref["sha"]


def test_divisao_linha_a_linha(corpus):
    """Line i of each file is in the validation bytes iff i % 20 == 0, each line once, in file order (Portuguese
    first), only lines below 3000; carregar_tudo keeps every line."""
    pasta, textos = corpus
    tr, val = DD.divide(pasta)
    tr_t, val_t = DD.divide(pasta, None)
    for lingua, ts in textos.items():
        for i, t in enumerate(ts):
            if not t:
                continue
            marca = f"[{lingua[0]}{i}] ".encode()
            dentro, fora = (val, tr) if i % 20 == 0 else (tr, val)
            if i < 3000:
                assert dentro.count(marca) == 1 and fora.count(marca) == 0, (lingua, i)
            else:
                assert tr.count(marca) == 0 and val.count(marca) == 0, (lingua, i)
            dentro_t = val_t if i % 20 == 0 else tr_t
            assert dentro_t.count(marca) == 1, (lingua, i)
    # bytes of a line: its text in UTF-8 and two newlines; the languages follow each other
    assert tr.startswith(textos["Portuguese"][1].encode() + b"\n\n" + textos["Portuguese"][2].encode() + b"\n\n")
    assert val.startswith(textos["Portuguese"][0].encode() + b"\n\n" + textos["Portuguese"][20].encode())
    p_ult = max(i for i in range(1, 3000) if i % 20 and textos["Portuguese"][i])
    assert tr.index(textos["Portuguese"][p_ult].encode()) < tr.index(b"[E1] ")


@pytest.mark.parametrize("caso", range(5))
def test_lote_vs_referencia(corpus, caso):
    g = json.load(open(GOLD))["lotes"][caso]
    tr, _ = DD.carregar(corpus[0])
    ger = torch.Generator().manual_seed(g["semente"])
    for ref in g["passos"]:
        est = ger.get_state()
        x, y = DD.lote(tr, ger, g["Bt"], g["T"])
        assert x.shape == (g["Bt"], g["T"]) and x.dtype == torch.int64
        assert _sha(x) == ref["x"] and _sha(y) == ref["y"] and x[0, :16].tolist() == ref["x0"]
        g2 = torch.Generator()
        g2.set_state(est)
        ini = DD.inicios(len(tr), g2, g["Bt"], g["T"])
        assert ini.tolist() == ref["ini"]
        # windows are the corpus slices at the starts, the targets shifted by one
        for b, s in enumerate(ini.tolist()):
            assert torch.equal(x[b], tr[s:s + g["T"]]) and torch.equal(y[b], tr[s + 1:s + g["T"] + 1])
        assert max(ini.tolist()) <= len(tr) - g["T"] - 2


def test_corpus_curto_e_bytes_invalidos():
    with pytest.raises(ValueError):
        DD.inicios(10, torch.Generator().manual_seed(0), 2, 9)
    with pytest.raises(ValueError):
        DD.Corpus(None, torch.tensor([0, 256]), dev="cpu")
    with pytest.raises(FileNotFoundError):
        os.environ.pop("JATAI_DADOS", None)
        DD.carregar()
