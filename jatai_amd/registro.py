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
    6: "invalid argument (token or target outside the vocabulary, or a corpus window past its end)",
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


class Cronometro:
    """GPU time per op over a step (`perfil`): a pair of events around each timed launch, read once per step."""

    def __init__(self):
        self.pares = []

    def abre(self, op):
        ini, fim = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ini.record()
        self.pares.append([op, ini, fim, False])

    def fecha_ultimo(self):
        if self.pares and not self.pares[-1][3]:
            self.pares[-1][2].record()
            self.pares[-1][3] = True

    def soma_em(self, tempos):
        """Adds this step's closed pairs to tempos (op -> [launches, ms]) and forgets them."""
        torch.cuda.synchronize()
        for op, ini, fim, fechado in self.pares:
            if fechado:
                ent = tempos.setdefault(op, [0, 0.0])
                ent[0] += 1
                ent[1] += ini.elapsed_time(fim)
        self.pares = []


def _problemas_tensor(t, dtype, papel):
    """What keeps one tensor from being a kernel operand: dtype, device, layout."""
    if not torch.is_tensor(t):
        return [f"{papel} is {type(t).__name__}, not a tensor"]
    p = []
    if t.dtype != dtype:
        p.append(f"{papel} {t.dtype}, expected {dtype}")
    if not t.is_cuda:
        p.append(f"{papel} not on the GPU")
    if not t.is_contiguous():
        p.append(f"{papel} not contiguous")
    return p


class Registro:
    # how each level of message is echoed: (stream or None, prefix); "erro" raises instead
    ECO = {"info": ("out", ""), "aviso": ("err", "[warning] "), "estatistica": (None, "")}

    def __init__(self, pasta, nome, lib=None, vigiar=False, perfil=False, eco=True):
        os.makedirs(pasta, exist_ok=True)
        self.pasta, self.nome, self.lib = pasta, nome, lib
        self.vigiar, self.perfil, self.eco = vigiar, perfil, eco
        self.diario = Diario(os.path.join(pasta, f"{nome}.jsonl"))
        self.escopo = []                 # current scope path, innermost last
        self.lancamentos = []            # Lancamento per launch id of the current step (or of a captured graph)
        self.passo = None
        self.cronometro = Cronometro()
        self.tempos = {}                 # op -> [launches, GPU ms] accumulated since the last report
        self.passos_medidos = 0
        self.ultimo_evento = None

    # ------------------------------------------------------------------ messages
    def onde(self):
        return " / ".join(self.escopo) or "-"

    def escreve(self, tipo, **kw):
        """One record of the run's log, stamped with the step and scope."""
        return self.diario.grava(tipo, self.passo, self.onde(), **kw)

    def _relata(self, nivel, msg, **kw):
        """Logs msg at a level; echoes info (when `eco`) and warnings; an error raises ErroJatai whose text leads with
        the step and the scope path, then the message."""
        self.escreve(nivel, msg=msg, **kw)
        if nivel == "erro":
            raise ErroJatai(f"step {self.passo}, {self.onde()}:\n{msg}")
        destino, prefixo = self.ECO[nivel]
        if destino == "err" or (destino == "out" and self.eco):
            print(f"{prefixo}{msg}" if destino == "out" else f"{prefixo}step {self.passo}, {self.onde()}: {msg}",
                  file=sys.stderr if destino == "err" else sys.stdout, flush=True)

    def info(self, msg, **kw):
        self._relata("info", msg, **kw)

    def aviso(self, msg, **kw):
        self._relata("aviso", msg, **kw)

    def falha(self, msg, **kw):
        self._relata("erro", msg, **kw)

    def exige(self, cond, msg):
        if not cond:
            self._relata("erro", msg)

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
        self.cronometro.pares = []
        if self.lib is not None:
            self.lib.jt_erro_limpa()

    def registra(self, op, entradas, forma_saida, tempo=True):
        """Records a launch and returns its id. tempo=False: a further id of a batched launch, whose time is
        counted under the batch's first id."""
        kid = len(self.lancamentos)
        self.lancamentos.append(Lancamento(kid, op, self.onde(), entradas, tuple(forma_saida) if forma_saida else None))
        if self.perfil and tempo:
            self.cronometro.abre(op)
        return kid

    def depois(self, kid, codigo):
        if self.perfil:
            self.cronometro.fecha_ultimo()
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
        """End of a step: the device record is read (an event raises), and with `perfil` the step's op times are
        added to the running totals."""
        if self.lib is not None:
            self.confere_device()
        if self.perfil:
            self.cronometro.soma_em(self.tempos)
            self.passos_medidos += 1

    def relatorio_tempos(self, passos=None):
        """Logs (and echoes) the GPU time per op since the last report -- launches and milliseconds per step,
        microseconds per launch, share and running share of the step -- and restarts the totals."""
        if not self.tempos:
            return None
        passos = passos or max(self.passos_medidos, 1)
        total = sum(ms for _, ms in self.tempos.values())
        tabela, acumulado = [], 0.0
        for op, (n, ms) in sorted(self.tempos.items(), key=lambda kv: -kv[1][1]):
            acumulado += ms
            tabela.append(dict(op=op, lancamentos_por_passo=n / passos, ms_por_passo=ms / passos, us_por_lancamento=1e3 * ms / n,
                               fracao=ms / total, fracao_acumulada=acumulado / total))
        texto = [f"GPU time over {passos} step(s): {total / passos:.3f} ms per step"]
        texto += [f"  {t['op']:28s} {t['lancamentos_por_passo']:6.1f} x {t['us_por_lancamento']:9.2f} us = {t['ms_por_passo']:8.3f} ms"
                  f"  {100 * t['fracao']:5.1f}%  (cum. {100 * t['fracao_acumulada']:5.1f}%)" for t in tabela]
        self.info("\n".join(texto), tempos=tabela)
        self.tempos, self.passos_medidos = {}, 0
        return tabela

    # ------------------------------------------------------------------ format guards
    def _formato(self, nome, m, E, tipo):
        """Block formats: mantissa `tipo` [R, C] with C a multiple of BLK, int8 exponents [R, C / BLK], both
        contiguous on the GPU (BLK read from jatai_amd.ops at call time)."""
        erros = _problemas_tensor(m, tipo, "mantissa") + _problemas_tensor(E, torch.int8, "exponent")
        if torch.is_tensor(m) and torch.is_tensor(E):
            if m.dim() != 2:
                erros.append(f"mantissa of {m.dim()} dimensions, expected 2")
            elif m.shape[1] % O.BLK:
                erros.append(f"{m.shape[1]} columns, not a multiple of BLK={O.BLK}")
            elif tuple(E.shape) != (m.shape[0], m.shape[1] // O.BLK):
                erros.append(f"exponent shape {tuple(E.shape)}, expected {(m.shape[0], m.shape[1] // O.BLK)}")
        if erros:
            self.falha(f"argument '{nome}': " + "; ".join(erros))

    def confere_bloco(self, nome, t):
        self._formato(nome, t[0], t[1], torch.int8)

    def confere_r16(self, nome, t):
        self._formato(nome, t[0], t[1], torch.int16)

    def confere_cru(self, nome, t):
        """Raw format: int32 accumulators and int16 exponents of one shape, contiguous on the GPU."""
        acc, e = t
        erros = _problemas_tensor(acc, torch.int32, "accumulator") + _problemas_tensor(e, torch.int16, "exponent")
        if torch.is_tensor(acc) and torch.is_tensor(e) and acc.shape != e.shape:
            erros.append(f"accumulator {tuple(acc.shape)} and exponent {tuple(e.shape)} shapes differ")
        if erros:
            self.falha(f"raw argument '{nome}': " + "; ".join(erros))

    # ------------------------------------------------------------------ statistics
    def estatistica(self, nome, t, zeros_normais=False):
        """How well a block tensor uses its format, logged as one record (torch reductions, off the hot path):
        share of zero blocks; over the other blocks, the exponent range and median, the mantissa bits the block
        maximum uses (7 when the quantization is normalized), the share of zero and of saturated (+-127)
        mantissas. Warns when every block is zero, when most mantissas of live blocks are zero (unless zeros are
        expected, as after ReLU), when a block maximum uses fewer than 6 bits, and when an exponent comes within
        16 of either end of the INT8 exponent range (-126 .. 126)."""
        m, E = t
        blocos = m.reshape(m.shape[0], -1, O.BLK)
        vivos = E != O.E_ZERO
        n_vivos = int(vivos.sum())
        rec = {"nome": nome, "blocos": int(E.numel()), "blocos_zero": round(1 - n_vivos / max(E.numel(), 1), 4)}
        if n_vivos:
            ev = E[vivos].to(torch.int32)
            mv = blocos[vivos].to(torch.int32)
            maior = mv.abs().amax(-1)
            bits = torch.where(maior > 0, torch.floor(torch.log2(maior.clamp(min=1).float())) + 1, torch.zeros_like(maior, dtype=torch.float32))
            rec.update(exp_min=int(ev.min()), exp_mediana=int(ev.median()), exp_max=int(ev.max()),
                       bits_usados=round(float(bits.mean()), 3), zeros_em_vivos=round(float((mv == 0).float().mean()), 4),
                       saturados=round(float((mv.abs() == 127).float().mean()), 5))
        self.escreve("estatistica", **rec)
        if not n_vivos:
            self.aviso(f"'{nome}': every block is zero")
            return rec
        if not zeros_normais and rec["zeros_em_vivos"] > 0.5:
            self.aviso(f"'{nome}': {rec['zeros_em_vivos']:.0%} of the mantissas of its live blocks are zero")
        if rec["bits_usados"] < 6:
            self.aviso(f"'{nome}': block maxima use {rec['bits_usados']:.2f} of 7 mantissa bits on average")
        if rec["exp_min"] < -110 or rec["exp_max"] > 110:
            self.aviso(f"'{nome}': exponents {rec['exp_min']} .. {rec['exp_max']}, within 16 of the INT8 exponent range")
        return rec
