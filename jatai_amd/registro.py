"""Launch registry of the INT8 training step: every kernel launch gets an id, and anything that goes wrong -- a
malformed tensor, a refused launch, an event a kernel raised on the device -- becomes one exception that says
what happened, in which op and scope, where in the output and with which value.

The parts:

  `Lancamento`  one record per launch, in launch order: id (its index), op name, scope path, inputs, output shape.
                The id travels to the kernel as its last argument (`kid`), so a device event names its record.
  `Evento`      the device's error record (the first event since the last clear: count, code, kid, flat index,
                value, extra datum; `jt_erro_le`), decoded against the launch records.
  `Diario`      the append-only JSONL log of a run (`<pasta>/<nome>.jsonl`).
  `Registro`    the object the operator layer and the model hold: format guards before a launch, the return code
                after it, the device record once per step (or after every launch with `vigiar`), per-op GPU time
                with `perfil`, and tensor statistics.

A device event saves the inputs of the launch that raised it (`<pasta>/falha_passo<P>_<kid>_<op>.pt`, a dict of
CPU tensors; load it with torch.load(..., weights_only=True)) so the event can be re-run, e.g. through the CPU
oracle. In a replayed graph the saved tensors are the graph's own buffers read after the replay: inputs that a
later kernel of the same step overwrites are saved as that kernel left them.

Interface kept from the reference's `Registro` (jatai_cuda/registro.py:42-221), because the operator layer and
the model code call it: registra / depois / confere_bloco / confere_cru / confere_r16 / exige / falha / trecho /
novo_passo / fim_passo / confere_device / relatorio_tempos / estatistica and the attributes lib, lancamentos,
vigiar, perfil. A device event's message carries the three lines callers match
(jatai_cuda/teste_erro_grafo.py:26): the scope path, "linha R, coluna C" and "valor    : V".
"""
import contextlib
import ctypes
import dataclasses
import json
import os
import sys
import time

import torch

from . import ops as O

# device event codes (csrc/jt_comum.h: E_ACUM .. E_ARG), as the kernels report them
EVENTOS = {
    1: "accumulator reached 2^30 (beyond the int32 range the format keeps)",
    2: "block exponent above 126 (INT8 exponent overflow)",
    3: "mantissa beyond +-127 after the exponent bump",
    4: "division by zero (softmax sum <= 0)",
    5: "left shift would lose bits (result >= 2^30)",
    6: "invalid argument (token or target outside the vocabulary)",
}


class ErroJatai(RuntimeError):
    pass


@dataclasses.dataclass
class Lancamento:
    kid: int
    op: str
    trecho: str
    entradas: dict
    forma: tuple


@dataclasses.dataclass
class Evento:
    """The first device event of a step, decoded."""
    n: int
    codigo: int
    kid: int
    idx: int
    valor: int
    aux: int
    lancamento: Lancamento = None
    arquivo: str = None

    def posicao(self):
        forma = self.lancamento.forma if self.lancamento else None
        if forma and len(forma) == 2 and forma[1]:
            return f"linha {self.idx // forma[1]}, coluna {self.idx % forma[1]} (forma {tuple(forma)})"
        return f"indice {self.idx}"

    def mensagem(self):
        l = self.lancamento
        return "\n".join([
            EVENTOS.get(self.codigo, f"device event code {self.codigo}"),
            f"  operacao : {l.op}",
            f"  trecho   : {l.trecho}",
            f"  posicao  : {self.posicao()}",
            f"  valor    : {self.valor}   (extra: {self.aux})",
            f"  eventos  : {self.n} this step (the first one is shown)",
            f"  entradas : {_formas(l.entradas)}",
            f"  salvas em: {self.arquivo}",
        ])


def _formas(ent):
    return {k: (tuple(v.shape) if torch.is_tensor(v) else v) for k, v in ent.items()}


class Diario:
    """Append-only JSONL log; each record carries the time, its type, the step and the scope."""

    def __init__(self, caminho):
        self.arq = open(caminho, "a")

    def grava(self, tipo, passo, trecho, **campos):
        rec = dict(hora=time.strftime("%H:%M:%S"), tipo=tipo, passo=passo, trecho=trecho, **campos)
        self.arq.write(json.dumps(rec, ensure_ascii=False, default=str) + "\n")
        self.arq.flush()
        return rec


class Registro:
    def __init__(self, pasta, nome, lib=None, vigiar=False, perfil=False, eco=True):
        os.makedirs(pasta, exist_ok=True)
        self.pasta, self.nome, self.lib = pasta, nome, lib
        self.vigiar, self.perfil, self.eco = vigiar, perfil, eco
        self.diario = Diario(os.path.join(pasta, f"{nome}.jsonl"))
        self.escopo = []                 # current scope path, innermost last
        self.lancamentos = []            # Lancamento per launch id of the current step (or of a captured graph)
        self.passo = None
        self._cronos = []                # (op, start event, end event) of the current step, with perfil
        self.tempos = {}                 # op -> accumulated GPU ms over the steps since the last report
        self.ultimo_evento = None

    # ------------------------------------------------------------------ log and failure
    def onde(self):
        return " / ".join(self.escopo) or "-"

    def escreve(self, tipo, **kw):
        return self.diario.grava(tipo, self.passo, self.onde(), **kw)

    def info(self, msg, **kw):
        self.escreve("info", msg=msg, **kw)
        if self.eco:
            print(msg, flush=True)

    def aviso(self, msg, **kw):
        self.escreve("aviso", msg=msg, **kw)
        print(f"[warning] step {self.passo} | {self.onde()} | {msg}", file=sys.stderr, flush=True)

    def falha(self, msg, **kw):
        self.escreve("erro", msg=msg, **kw)
        raise ErroJatai(f"\n[ERRO] passo {self.passo} | {self.onde()}\n{msg}")

    def exige(self, cond, msg):
        if not cond:
            self.falha(msg)

    @contextlib.contextmanager
    def trecho(self, nome):
        self.escopo.append(nome)
        try:
            yield
        finally:
            self.escopo.pop()

    # ------------------------------------------------------------------ steps and launches
    def novo_passo(self, passo):
        self.passo = passo
        self.lancamentos = []
        self._cronos = []
        if self.lib is not None:
            self.lib.jt_erro_limpa()

    def registra(self, op, entradas, forma_saida, tempo=True):
        """Records a launch and returns its id. tempo=False: a further id of a batched launch, whose time is
        counted under the batch's first id."""
        kid = len(self.lancamentos)
        self.lancamentos.append(Lancamento(kid, op, self.onde(), entradas, tuple(forma_saida) if forma_saida else None))
        if self.perfil and tempo:
            par = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            par[0].record()
            self._cronos.append((op, *par))
        return kid

    def depois(self, kid, codigo):
        if self.perfil and self._cronos:
            self._cronos[-1][2].record()
        if codigo != 0:
            l = self.lancamentos[kid]
            self.falha(f"the HIP runtime refused the launch of '{l.op}' (hipError {codigo}); inputs {_formas(l.entradas)}")
        if self.vigiar:
            self.confere_device()

    def _le_device(self):
        buf = (ctypes.c_longlong * 6)()
        n = self.lib.jt_erro_le(buf)
        if n < 0:
            ult = self.lancamentos[-1] if self.lancamentos else None
            self.falha(f"reading the device error record failed (hipError {-n}): an earlier kernel probably aborted; "
                       f"last launch {ult.op + ' in ' + ult.trecho if ult else '-'}")
        return Evento(*[int(x) for x in buf]) if n > 0 else None

    def _salva(self, ev):
        l = ev.lancamento
        arq = os.path.join(self.pasta, f"falha_passo{self.passo}_{l.kid}_{l.op.replace('+', '_')}.pt")
        try:
            torch.save({k: (v.detach().cpu() if torch.is_tensor(v) else v) for k, v in l.entradas.items()}, arq)
            return arq
        except Exception as e:          # the save must not hide the event itself
            return f"(not saved: {e})"

    def confere_device(self):
        """Reads the device error record (synchronizes the device); a recorded event raises ErroJatai."""
        ev = self._le_device()
        if ev is None:
            return
        if not 0 <= ev.kid < len(self.lancamentos):
            self.falha(f"{EVENTOS.get(ev.codigo, ev.codigo)} in an unknown launch id {ev.kid} (index {ev.idx}, value {ev.valor})")
        ev.lancamento = self.lancamentos[ev.kid]
        ev.arquivo = self._salva(ev)
        self.ultimo_evento = ev
        self.escopo = [ev.lancamento.trecho]
        self.falha(ev.mensagem(), codigo=ev.codigo, op=ev.lancamento.op, idx=ev.idx, valor=ev.valor, aux=ev.aux, arquivo=ev.arquivo)

    def fim_passo(self):
        if self.lib is not None:
            self.confere_device()
        if self.perfil:
            torch.cuda.synchronize()
            for op, a, b in self._cronos:
                self.tempos[op] = self.tempos.get(op, 0.0) + a.elapsed_time(b)

    def relatorio_tempos(self, passos):
        if not self.tempos:
            return
        tot = sum(self.tempos.values())
        ordem = sorted(self.tempos.items(), key=lambda kv: -kv[1])
        linhas = [f"  {op:24s} {ms / passos:8.3f} ms/step  {100 * ms / tot:5.1f}%" for op, ms in ordem]
        self.info("GPU time per op:\n" + "\n".join(linhas) + f"\n  {'total':24s} {tot / passos:8.3f} ms/step",
                  tempos={k: v / passos for k, v in self.tempos.items()})
        self.tempos = {}

    # ------------------------------------------------------------------ format guards
    def _formato(self, nome, m, E, tipo):
        """Block formats: mantissa `tipo` [R, C] with C a multiple of BLK, int8 exponents [R, C / BLK], both
        contiguous on the GPU (BLK read from jatai_amd.ops at call time)."""
        erros = []
        if m.dtype != tipo:
            erros.append(f"mantissa {m.dtype}, expected {tipo}")
        if E.dtype != torch.int8:
            erros.append(f"exponent {E.dtype}, expected int8")
        if not (m.is_cuda and E.is_cuda):
            erros.append("not on the GPU")
        if not (m.is_contiguous() and E.is_contiguous()):
            erros.append("not contiguous")
        if m.dim() != 2:
            erros.append(f"mantissa of {m.dim()} dimensions, expected 2")
        elif m.shape[1] % O.BLK:
            erros.append(f"{m.shape[1]} columns, not a multiple of BLK={O.BLK}")
        elif tuple(E.shape) != (m.shape[0], m.shape[1] // O.BLK):
            erros.append(f"exponent shape {tuple(E.shape)}, expected {(m.shape[0], m.shape[1] // O.BLK)}")
        if erros:
            self.falha(f"argument '{nome}': " + "; ".join(erros))

    def confere_bloco(self, nome, t):
        m, E = t
        if not (torch.is_tensor(m) and torch.is_tensor(E)):
            self.falha(f"argument '{nome}': expected a (mantissa, exponent) pair of tensors, got {type(m)}, {type(E)}")
        self._formato(nome, m, E, torch.int8)

    def confere_r16(self, nome, t):
        self._formato(nome, t[0], t[1], torch.int16)

    def confere_cru(self, nome, t):
        acc, e = t
        erros = []
        if acc.dtype != torch.int32:
            erros.append(f"accumulator {acc.dtype}, expected int32")
        if e.dtype != torch.int16:
            erros.append(f"exponent {e.dtype}, expected int16")
        if acc.shape != e.shape:
            erros.append(f"shapes differ: {tuple(acc.shape)} and {tuple(e.shape)}")
        if not (acc.is_cuda and acc.is_contiguous() and e.is_contiguous()):
            erros.append("not on the GPU or not contiguous")
        if erros:
            self.falha(f"raw argument '{nome}': " + "; ".join(erros))

    # ------------------------------------------------------------------ statistics
    def estatistica(self, nome, t, zeros_normais=False):
        """Summary of a block tensor, logged (torch reductions outside the hot path); warns on the patterns that
        precede trouble: a tensor rounded to zero, a majority of zero mantissas, exponents near -126."""
        m, E = t
        vivos = E != O.E_ZERO
        nz = bool(vivos.any())
        rec = {
            "nome": nome,
            "zeros": round(float((m == 0).float().mean()), 4),
            "blocos_zerados": round(float((~vivos).float().mean()), 4),
            "exp_min": int(E[vivos].min()) if nz else None,
            "exp_max": int(E[vivos].max()) if nz else None,
            "maior_mantissa_media": round(float(m.abs().reshape(m.shape[0], -1, O.BLK).amax(-1).float().mean()), 1),
        }
        self.escreve("estatistica", **rec)
        if not nz:
            self.aviso(f"'{nome}' is all zero")
        elif not zeros_normais and rec["zeros"] > 0.5:
            self.aviso(f"'{nome}' has {rec['zeros']:.0%} zero mantissas: small values lost to rounding?")
        if rec["exp_min"] is not None and rec["exp_min"] < -110:
            self.aviso(f"'{nome}' has exponent {rec['exp_min']}, close to the INT8 limit -126")
        return rec
