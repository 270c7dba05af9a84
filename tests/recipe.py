"""Portable, seeded input recipes for parity tests and golden fixtures.

Every input is drawn from a SplitMix64 stream (Steele, Lea & Flood, "Fast splittable pseudorandom number
generators", OOPSLA 2014) written in numpy uint64 arithmetic, so the same seed gives the same bytes on any
machine and any numpy/torch version. The distributions mirror the reference's test generators
(`jatai_cuda/teste_ops.py:18-31`: `bloco` and `cru`), re-stated with this stream instead of torch's RNG.
"""
import hashlib

import numpy as np

E_ZERO = -127
_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def splitmix64(seed, n):
    """n consecutive SplitMix64 outputs (uint64) for a given seed."""
    idx = np.arange(1, n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + idx * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    return z


def substream(seed, tag):
    """Derive an independent seed from (seed, tag) via SHA-256 (tag: str)."""
    h = hashlib.sha256(f"{seed}:{tag}".encode()).digest()
    return int.from_bytes(h[:8], "little")


def uniform_int(seed, shape, lo, hi):
    """Integers uniform in [lo, hi] (inclusive), int64."""
    n = int(np.prod(shape)) if len(shape) else 1
    x = splitmix64(seed, n) >> np.uint64(11)
    span = np.uint64(hi - lo + 1)
    return (x % span).astype(np.int64).reshape(shape) + lo


def uniform01(seed, shape):
    n = int(np.prod(shape)) if len(shape) else 1
    x = splitmix64(seed, n) >> np.uint64(11)
    return (x.astype(np.float64) / float(1 << 53)).reshape(shape)


def normal32(seed, shape, sigma=1.0):
    """float32 samples of N(0, sigma^2) (Box-Muller on two uniform streams, in float64, rounded once)."""
    u1 = uniform01(substream(seed, "u1"), shape)
    u2 = uniform01(substream(seed, "u2"), shape)
    z = np.sqrt(-2.0 * np.log1p(-u1)) * np.cos(2.0 * np.pi * u2)
    return np.ascontiguousarray((sigma * z).astype(np.float32))


def bloco(seed, R, C, blk, espalha=4, zera=0.0, e0=-10, mmax=127):
    """Block tensor (m int8 [R,C], E int8 [R,C/blk]): mantissas uniform in [-mmax, mmax], exponents e0 +
    uniform[-espalha, espalha], and each block zeroed (m = 0, E = -127) with probability `zera`.
    Same distribution as `bloco()` in jatai_cuda/teste_ops.py:18-25."""
    m = uniform_int(substream(seed, "m"), (R, C), -mmax, mmax).astype(np.int8)
    E = (e0 + uniform_int(substream(seed, "E"), (R, C // blk), -espalha, espalha)).astype(np.int8)
    if zera:
        z = uniform01(substream(seed, "z"), (R, C // blk)) < zera
        m = m.reshape(R, C // blk, blk)
        m[z] = 0
        m = m.reshape(R, C)
        E[z] = E_ZERO
    return np.ascontiguousarray(m), np.ascontiguousarray(E)


def cru(seed, R, C, bits=24, e0=-30):
    """Raw tensor (acc int32 [R,C], e int16 [R,C]): acc uniform in [-2^bits, 2^bits - 1], e = e0 + uniform[-3, 3].
    Same distribution as `cru()` in jatai_cuda/teste_ops.py:28-31."""
    acc = uniform_int(substream(seed, "acc"), (R, C), -(1 << bits), (1 << bits) - 1).astype(np.int32)
    e = (e0 + uniform_int(substream(seed, "e"), (R, C), -3, 3)).astype(np.int16)
    return np.ascontiguousarray(acc), np.ascontiguousarray(e)


def tokens(seed, n, V):
    return uniform_int(seed, (n,), 0, V - 1).astype(np.int32)


def sha(a):
    """SHA-256 of an array's C-contiguous little-endian bytes (dtype fixed by the caller)."""
    a = np.ascontiguousarray(a)
    return hashlib.sha256(a.tobytes()).hexdigest()


# words of the synthetic byte corpus: 1- to 4-byte UTF-8 characters, JSON escapes (quote, backslash, newline, tab)
_PALAVRAS = ("o", "a", "de", "que", "não", "ação", "coração", "está", "você", "pão", "the", "of", "and", "naïve",
             "café", "über", "€5", "日本語", "한국어", "😀", "🚀ok", 'aspas "x"', "barra \\ y", "linha\nnova", "tab\tz",
             "ñ", "ß", "Ωμέγα", "—", "…", "123", "")


def corpus_sintetico(pasta, semente=1, linhas=(("Portuguese", 3012), ("English", 57))):
    """Writes Portuguese.jsonl and English.jsonl (one {"text": ...} per line, as the reference's corpus) into `pasta`
    and returns the texts per language. Line i of a file starts with "[<first letter><i>]"; its length and words
    come from a SplitMix64 stream; every 97th line is empty text. Lines past 3000 exercise carregar's limit."""
    import json
    import os
    textos = {}
    for lingua, n in linhas:
        s = substream(semente, "corpus:" + lingua)
        tam = uniform_int(substream(s, "tam"), (n,), 0, 40)
        pal = uniform_int(substream(s, "pal"), (n, 40), 0, len(_PALAVRAS) - 1)
        ts = []
        for i in range(n):
            corpo = " ".join(_PALAVRAS[p] for p in pal[i, :tam[i]])
            ts.append("" if i % 97 == 5 else f"[{lingua[0]}{i}] {corpo}")
        with open(os.path.join(pasta, f"{lingua}.jsonl"), "w", encoding="utf-8") as f:
            for t in ts:
                f.write(json.dumps({"text": t, "id": len(t)}, ensure_ascii=(len(t) % 2 == 0)) + "\n")
        textos[lingua] = ts
    return textos
