"""CPU oracle for the GGUF quantized linear path: GGML block codecs in numpy.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module, and only as the checker (or the timed CPU
baseline), never as a code path of the product.  The product (``gguf_hip``) fails loudly
when its HIP library is missing; it never falls back to this file.

What it restates.  The reference dequantizer of this path is gguf-py 0.17.1
(``gguf.quants.dequantize``; pinned at ``gguf-plugin/requirements.txt:1``, called at
``gguf-plugin/test_gguf_rco_cpu.py:347-353`` and ``gguf-plugin/patches/gguf-prefill-dispatch.patch:42-45``).
gguf-py is not vendored in the reference and is absent here, so each codec below restates its
published algorithm, following the reference's own restatements where they exist:

* Q8_0 / Q3_K / Q5_K / Q6_K field parsing: ``gguf-plugin/gluon/kq_ref.py:30-80``;
  operation order ``gguf-plugin/gluon/kq_ref.py:83-91``; ``get_scale_min_k4``
  ``gguf-plugin/gluon/kq_ref.py:17-27``.
* Q4_K: ``gguf-plugin/gluon/q4k.py:5-20``.
* Q2_K: ``gguf-plugin/gluon/q2k.py:5-12`` (bit and scale-byte mapping).
* IQ4_XS: ``gguf-plugin/gluon/iq4xs.py:5-11`` (+ ``KVALUES`` ``:36``).
* IQ3_S: ``gguf-plugin/gluon/iq3s_tile_dequant.py:30-53`` (fields, grid index, sign bit,
  ``d * (1 + 2 s) * g`` and its power-of-two equivalence with the CUDA form) and the field
  offsets of ``gguf-plugin/test_gguf_rco_cpu.py:215-227``.
* Q4_0 / Q5_0 / IQ4_NL: not written out anywhere in the reference (served there only by the
  unvendored CUDA MMVQ, ``gguf-plugin/patches/gguf-mmvq-batched.patch:98-126,258-266``); restated
  from the GGML block spec.  Their parity with gguf-py is pinned by hand-computed known-answer
  blocks and brute force in ``tests/test_oracle.py`` (no reference vector exists for them).

Bit-exactness argument (why any IEEE evaluation order gives gguf-py's fp32 bits): every
product ``d * sc * q`` and ``dmin * m`` has at most 24 significant bits (fp16 d: 11, integer
sub-scales: <= 7, q: <= 8), so it is exact in fp32; only the K-quant min subtraction
(Q2_K / Q4_K / Q5_K) rounds, once.  ``dequantize(..., f64=True)`` computes the same values in
float64 so the tests can assert ``fp32 == float32(fp64)`` for every type.
"""
from __future__ import annotations

import numpy as np

from .tables import IQ3S_GRID_BYTES, IQ4_KVALUES

# GGML type ids (ggml.h enum; Q8_0/Q3_K/Q5_K/Q6_K/Q4_K/Q2_K/IQ4_XS/IQ3_S also at
# gguf-plugin/gluon/interface.py:28-35 and gguf-plugin/gluon/kq_tiles.py:21)
Q4_0, Q5_0, Q8_0 = 2, 6, 8
Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 10, 11, 12, 13, 14
IQ4_NL, IQ3_S, IQ4_XS = 20, 21, 23

# type -> (name, weights per block, bytes per block)  (gguf.GGML_QUANT_SIZES)
TYPES = {
    Q4_0: ("Q4_0", 32, 18),
    Q5_0: ("Q5_0", 32, 22),
    Q8_0: ("Q8_0", 32, 34),
    Q2_K: ("Q2_K", 256, 84),
    Q3_K: ("Q3_K", 256, 110),
    Q4_K: ("Q4_K", 256, 144),
    Q5_K: ("Q5_K", 256, 176),
    Q6_K: ("Q6_K", 256, 210),
    IQ4_NL: ("IQ4_NL", 32, 18),
    IQ3_S: ("IQ3_S", 256, 110),
    IQ4_XS: ("IQ4_XS", 256, 136),
}
NAMES = {t: v[0] for t, v in TYPES.items()}
ALL_TYPES = tuple(TYPES)


def row_bytes(wt: int, K: int) -> int:
    _, bw, bb = TYPES[wt]
    assert K % bw == 0, (wt, K)
    return K // bw * bb


def _f16(b: np.ndarray, dt) -> np.ndarray:
    """Two little-endian bytes (last axis) -> fp16 value as dt."""
    return np.ascontiguousarray(b).view(np.float16)[..., 0].astype(dt)


def _scale_min_k4(s12: np.ndarray):
    """The 12 packed scale bytes of Q4_K / Q5_K -> (sc[8], m[8]), 6 bits each
    (gguf-plugin/gluon/kq_ref.py:17-27)."""
    s = s12.astype(np.int32)
    sc = np.empty(s.shape[:-1] + (8,), np.int32)
    mn = np.empty_like(sc)
    for j in range(4):
        sc[..., j] = s[..., j] & 63
        mn[..., j] = s[..., j + 4] & 63
        sc[..., j + 4] = (s[..., j + 8] & 0xF) | ((s[..., j] >> 6) << 4)
        mn[..., j + 4] = (s[..., j + 8] >> 4) | ((s[..., j + 4] >> 6) << 4)
    return sc, mn


def _nib32(qs: np.ndarray) -> np.ndarray:
    """[..., 16] bytes -> [..., 32]: low nibbles are weights 0..15, high nibbles 16..31."""
    q = qs.astype(np.int32)
    return np.concatenate([q & 0xF, q >> 4], axis=-1)


def fields(raw: np.ndarray, wt: int, K: int) -> dict:
    """Parse rows of blocks into integer fields.

    Returns ``q`` int32 [n, K] (the integer the weight is a multiple of, with the format's
    offset applied: Q4_0 nib-8, Q6_K u-32, IQ4 kvalue, IQ3_S +-grid), ``sc`` the fp16-free
    integer scale per group of ``G`` weights [n, K // G] (1 where the format has none),
    ``d`` fp16 bits as float per group's super-block [n, K // G], and, for Q2_K/Q4_K/Q5_K,
    ``m`` int [n, K // G] and ``dmin`` [n, K // G].  value = d * sc * q - dmin * m.
    """
    raw = np.ascontiguousarray(raw)
    n = raw.shape[0]
    _, bw, bb = TYPES[wt]
    nblk = K // bw
    b = raw.reshape(n, nblk, bb)
    out = {}
    if wt in (Q4_0, IQ4_NL):                       # d | qs[16]
        d = _f16(b[..., 0:2], np.float64)
        nib = _nib32(b[..., 2:18])
        q = nib - 8 if wt == Q4_0 else IQ4_KVALUES.astype(np.int32)[nib]
        out.update(q=q.reshape(n, K), G=32, d=d, sc=np.ones_like(d, dtype=np.int32))
    elif wt == Q5_0:                               # d | qh u32 | qs[16]
        d = _f16(b[..., 0:2], np.float64)
        qh = np.ascontiguousarray(b[..., 2:6]).view(np.uint32)[..., 0].astype(np.int64)
        hb = (qh[..., None] >> np.arange(32)) & 1
        q = (_nib32(b[..., 6:22]) | (hb << 4).astype(np.int32)) - 16
        out.update(q=q.reshape(n, K), G=32, d=d, sc=np.ones_like(d, dtype=np.int32))
    elif wt == Q8_0:                               # d | int8 qs[32]
        d = _f16(b[..., 0:2], np.float64)
        q = np.ascontiguousarray(b[..., 2:34]).view(np.int8).astype(np.int32)
        out.update(q=q.reshape(n, K), G=32, d=d, sc=np.ones_like(d, dtype=np.int32))
    elif wt == Q2_K:                               # scales[16] | qs[64] | d | dmin
        sc_b = b[..., 0:16].astype(np.int32)
        qs = b[..., 16:80].astype(np.int32)
        d = _f16(b[..., 80:82], np.float64)
        dmin = _f16(b[..., 82:84], np.float64)
        q = np.empty((n, nblk, 256), np.int32)
        for w in range(256):                       # w = 128 h + 32 t + l: bits 2t of byte 32h + l
            h, t, l = w // 128, (w // 32) % 4, w % 32
            q[..., w] = (qs[..., 32 * h + l] >> (2 * t)) & 3
        out.update(q=q.reshape(n, K), G=16, sc=(sc_b & 0xF).reshape(n, -1), m=(sc_b >> 4).reshape(n, -1),
                   d=np.repeat(d, 16, axis=-1).reshape(n, -1), dmin=np.repeat(dmin, 16, axis=-1).reshape(n, -1))
    elif wt == Q3_K:                               # hmask[32] | qs[64] | scales[12] | d
        hm = b[..., 0:32].astype(np.int32)
        qs = b[..., 32:96].astype(np.int32)
        s = b[..., 96:108].astype(np.int32)
        d = _f16(b[..., 108:110], np.float64)
        q = np.empty((n, nblk, 256), np.int32)
        for w in range(256):
            h, j, l = w // 128, (w // 32) % 4, w % 32
            hb = (hm[..., l] >> (4 * h + j)) & 1
            q[..., w] = ((qs[..., 32 * h + l] >> (2 * j)) & 3) - np.where(hb == 1, 0, 4)
        sc = np.empty((n, nblk, 16), np.int32)
        for i in range(16):
            lo = (s[..., i % 8] >> (4 * (i // 8))) & 0xF
            hi = (s[..., 8 + i % 4] >> (2 * (i // 4))) & 3
            sc[..., i] = (lo | (hi << 4)) - 32
        out.update(q=q.reshape(n, K), G=16, sc=sc.reshape(n, -1), d=np.repeat(d, 16, axis=-1).reshape(n, -1))
    elif wt in (Q4_K, Q5_K):                       # d | dmin | scales[12] | (qh[32]) | qs[128]
        d = _f16(b[..., 0:2], np.float64)
        dmin = _f16(b[..., 2:4], np.float64)
        sc, mn = _scale_min_k4(b[..., 4:16])
        qs = b[..., 16:144].astype(np.int32) if wt == Q4_K else b[..., 48:176].astype(np.int32)
        q = np.empty((n, nblk, 256), np.int32)
        for w in range(256):                       # sub-block ib = w // 32: nibble 4 (ib & 1) of byte 32 (ib >> 1) + p
            ib, p = w // 32, w % 32
            q[..., w] = (qs[..., 32 * (ib >> 1) + p] >> (4 * (ib & 1))) & 0xF
            if wt == Q5_K:
                q[..., w] |= ((b[..., 16 + p].astype(np.int32) >> ib) & 1) << 4
        out.update(q=q.reshape(n, K), G=32, sc=sc.reshape(n, -1), m=mn.reshape(n, -1),
                   d=np.repeat(d, 8, axis=-1).reshape(n, -1), dmin=np.repeat(dmin, 8, axis=-1).reshape(n, -1))
    elif wt == Q6_K:                               # ql[128] | qh[64] | int8 scales[16] | d
        ql = b[..., 0:128].astype(np.int32)
        qh = b[..., 128:192].astype(np.int32)
        sc = np.ascontiguousarray(b[..., 192:208]).view(np.int8).astype(np.int32)
        d = _f16(b[..., 208:210], np.float64)
        q = np.empty((n, nblk, 256), np.int32)
        for w in range(256):
            h, t, p = w // 128, (w // 32) % 4, w % 32
            lo = (ql[..., 64 * h + 32 * (t & 1) + p] >> (4 * (t >> 1))) & 0xF
            hi = (qh[..., 32 * h + p] >> (2 * t)) & 3
            q[..., w] = (lo | (hi << 4)) - 32
        out.update(q=q.reshape(n, K), G=16, sc=sc.reshape(n, -1), d=np.repeat(d, 16, axis=-1).reshape(n, -1))
    elif wt == IQ4_XS:                             # d | scales_h u16 | scales_l[4] | qs[128]
        d = _f16(b[..., 0:2], np.float64)
        sh = np.ascontiguousarray(b[..., 2:4]).view(np.uint16)[..., 0].astype(np.int32)
        sl = b[..., 4:8].astype(np.int32)
        ls = np.empty((n, nblk, 8), np.int32)
        for ib in range(8):
            ls[..., ib] = ((sl[..., ib // 2] >> (4 * (ib % 2))) & 0xF) | (((sh >> (2 * ib)) & 3) << 4)
        nib = _nib32(b[..., 8:136].reshape(n, nblk, 8, 16))             # [n, nblk, 8, 32]
        q = IQ4_KVALUES.astype(np.int32)[nib]
        out.update(q=q.reshape(n, K), G=32, sc=(ls - 32).reshape(n, -1), d=np.repeat(d, 8, axis=-1).reshape(n, -1))
    elif wt == IQ3_S:                              # d | qs[64] | qh[8] | signs[32] | scales[4]
        d = _f16(b[..., 0:2], np.float64)
        qs = b[..., 2:66].astype(np.int32)
        qh = b[..., 66:74].astype(np.int32)
        sg = b[..., 74:106].astype(np.int32)
        scb = b[..., 106:110].astype(np.int32)
        q = np.empty((n, nblk, 256), np.int32)
        grid = IQ3S_GRID_BYTES.astype(np.int32)
        for j in range(256):                       # iq3s_tile_dequant.py:31-45
            ib, il, jj = j // 32, (j % 32) // 8, j % 8
            half, k4 = jj // 4, jj % 4
            idx = qs[..., 8 * ib + 2 * il + half] | ((qh[..., ib] << (8 - 2 * il - half)) & 256)
            g = grid[idx, k4]
            neg = (sg[..., 4 * ib + il] >> jj) & 1
            q[..., j] = np.where(neg == 1, -g, g)
        s = np.empty((n, nblk, 8), np.int32)
        for ib in range(8):
            s[..., ib] = (scb[..., ib // 2] >> (4 * (ib % 2))) & 0xF
        out.update(q=q.reshape(n, K), G=32, sc=(1 + 2 * s).reshape(n, -1), d=np.repeat(d, 8, axis=-1).reshape(n, -1))
    else:
        raise NotImplementedError(f"GGML type {wt}")
    return out


def dequantize(raw: np.ndarray, wt: int, K: int | None = None, f64: bool = False) -> np.ndarray:
    """uint8 rows [n, row_bytes] of GGML type ``wt`` -> weights [n, K] (fp32, or fp64 with f64).

    fp32: the operations gguf-py performs, in its order: ``(d * sc)`` then ``* q`` then
    ``- dmin * m`` (gguf-plugin/gluon/kq_ref.py:83-91), each an fp32 op.
    """
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    if raw.ndim == 1:
        raw = raw[None]
    _, bw, bb = TYPES[wt]
    if K is None:
        K = raw.shape[1] // bb * bw
    assert raw.shape[1] == K // bw * bb, (raw.shape, wt, K)
    f = fields(raw, wt, K)
    n, G = raw.shape[0], f["G"]
    dt = np.float64 if f64 else np.float32
    q = f["q"].astype(dt).reshape(n, K // G, G)
    dl = (f["d"].astype(dt) * f["sc"].astype(dt))[..., None]
    w = dl * q
    if "m" in f:
        w = w - (f["dmin"].astype(dt) * f["m"].astype(dt))[..., None]
    return w.reshape(n, K)


# ---------------------------------------------------------------------------------------
# Block generators (synthetic inputs).  Parity is on dequantization, so the quantizers only
# have to emit valid blocks of sensible magnitude; they follow GGML's simple reference
# quantizers where BASELINE names one (Q8_0: d = absmax / 127, round half away).

def _f16_bytes(v: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(v.astype(np.float16)).view(np.uint8).reshape(v.shape + (2,))


def _roundf(x: np.ndarray) -> np.ndarray:
    """Round half away from zero (gguf-py's np_roundf / C roundf)."""
    return np.sign(x) * np.floor(np.abs(x) + 0.5)


def random_blocks(rng: np.random.Generator, n: int, K: int, wt: int, dscale: float = 2.0 ** -8) -> np.ndarray:
    """Random valid rows: every bit pattern of the quantized fields is valid, so the bytes are
    uniform except the fp16 scale fields, which get finite positive values of magnitude
    ``dscale`` (the pattern of gguf-plugin/gluon/kq_ref.py:94-112).  IQ3_S / IQ4_XS d follow
    |N(0, 1e-3)|."""
    _, bw, bb = TYPES[wt]
    nblk = K // bw
    raw = rng.integers(0, 256, size=(n, nblk, bb), dtype=np.uint8)

    def dvals(scale=dscale):
        return rng.uniform(0.25, 1.0, size=(n, nblk)) * scale

    if wt in (Q4_0, Q5_0, Q8_0, IQ4_NL):
        raw[..., 0:2] = _f16_bytes(dvals(2.0 ** -6))
    elif wt == Q2_K:
        raw[..., 80:82] = _f16_bytes(dvals())
        raw[..., 82:84] = _f16_bytes(dvals())
    elif wt == Q3_K:
        raw[..., 108:110] = _f16_bytes(dvals())
    elif wt in (Q4_K, Q5_K):
        raw[..., 0:2] = _f16_bytes(dvals())
        raw[..., 2:4] = _f16_bytes(dvals())
    elif wt == Q6_K:
        raw[..., 208:210] = _f16_bytes(dvals())
    elif wt in (IQ4_XS, IQ3_S):
        raw[..., 0:2] = _f16_bytes(np.abs(rng.normal(0.0, 1e-3, size=(n, nblk))))
    return raw.reshape(n, nblk * bb)


def quantize(W: np.ndarray, wt: int) -> np.ndarray:
    """fp32 weights [n, K] -> GGML blocks [n, row_bytes] (simple round-to-nearest quantizers)."""
    W = np.ascontiguousarray(W, dtype=np.float32)
    n, K = W.shape
    _, bw, bb = TYPES[wt]
    nblk = K // bw
    x = W.reshape(n, nblk, bw)
    out = np.zeros((n, nblk, bb), np.uint8)
    if wt == Q8_0:
        d = np.abs(x).max(-1) / 127.0
        with np.errstate(divide="ignore"):
            idv = np.where(d == 0, 0.0, 1.0 / d)
        q = _roundf(x * idv[..., None]).astype(np.int8)
        out[..., 0:2] = _f16_bytes(d)
        out[..., 2:34] = q.view(np.uint8)
    elif wt in (Q4_0, Q5_0):
        nl = 8 if wt == Q4_0 else 16
        imax = np.abs(x).argmax(-1)
        mx = np.take_along_axis(x, imax[..., None], -1)[..., 0]
        d = mx / -nl
        with np.errstate(divide="ignore"):
            idv = np.where(d == 0, 0.0, 1.0 / d)
        q = np.clip(np.trunc(x * idv[..., None] + nl + 0.5), 0, 2 * nl - 1).astype(np.int32)
        out[..., 0:2] = _f16_bytes(d)
        lo, hi = q[..., :16], q[..., 16:]
        if wt == Q4_0:
            out[..., 2:18] = ((lo & 0xF) | ((hi & 0xF) << 4)).astype(np.uint8)
        else:
            qh = np.zeros((n, nblk), np.uint64)
            for j in range(32):
                qh |= ((q[..., j] >> 4) & 1).astype(np.uint64) << np.uint64(j)
            out[..., 2:6] = qh.astype(np.uint32).view(np.uint8).reshape(n, nblk, 4)
            out[..., 6:22] = ((lo & 0xF) | ((hi & 0xF) << 4)).astype(np.uint8)
    elif wt in (IQ4_NL, IQ4_XS):
        kv = IQ4_KVALUES.astype(np.float32)
        G = 32
        xs = x.reshape(n, -1, G)
        imax = np.abs(xs).argmax(-1)
        mx = np.take_along_axis(xs, imax[..., None], -1)[..., 0]
        dsub = mx / kv[0]                                           # the extreme value lands on -127
        if wt == IQ4_XS:
            d = np.abs(dsub).reshape(n, nblk, 8).max(-1) / 31.0 * np.float32(1.0)
            d16 = d.astype(np.float16).astype(np.float32)
            with np.errstate(divide="ignore", invalid="ignore"):
                ls = np.where(d16[..., None] == 0, 0, np.clip(_roundf(dsub.reshape(n, nblk, 8) / d16[..., None]), -32, 31)).astype(np.int32)
            dl = (d16[..., None] * ls).reshape(n, -1)
        else:
            d16 = dsub.astype(np.float16).astype(np.float32)
            dl = d16
        with np.errstate(divide="ignore", invalid="ignore"):
            t = np.where(dl[..., None] == 0, 0.0, xs / dl[..., None])
        idx = np.abs(t[..., None] - kv).argmin(-1).astype(np.int32)  # nearest table value
        packed = (idx[..., :16] | (idx[..., 16:] << 4)).astype(np.uint8)
        if wt == IQ4_NL:
            out[..., 0:2] = _f16_bytes(d16)
            out[..., 2:18] = packed
        else:
            out[..., 0:2] = _f16_bytes(d16)
            u = (ls + 32).astype(np.int64)
            sh = np.zeros((n, nblk), np.int64)
            for ib in range(8):
                sh |= ((u[..., ib] >> 4) & 3) << (2 * ib)
            out[..., 2:4] = sh.astype(np.uint16).view(np.uint8).reshape(n, nblk, 2)
            for i in range(4):
                out[..., 4 + i] = ((u[..., 2 * i] & 0xF) | ((u[..., 2 * i + 1] & 0xF) << 4)).astype(np.uint8)
            out[..., 8:136] = packed.reshape(n, nblk, 128)
    elif wt in (Q2_K, Q4_K, Q5_K):
        G = 16 if wt == Q2_K else 32
        qmax = {Q2_K: 3, Q4_K: 15, Q5_K: 31}[wt]
        smax = 15 if wt == Q2_K else 63
        xs = x.reshape(n, nblk, 256 // G, G)
        lo = np.minimum(xs.min(-1), 0.0)
        hi = xs.max(-1)
        scale = (hi - lo) / qmax
        mins = -lo
        d = scale.max(-1) / smax
        dmin = mins.max(-1) / smax
        d16 = d.astype(np.float16).astype(np.float32)
        dm16 = dmin.astype(np.float16).astype(np.float32)
        with np.errstate(divide="ignore", invalid="ignore"):
            isc = np.where(d16[..., None] == 0, 0, np.clip(_roundf(scale / d16[..., None]), 0, smax)).astype(np.int32)
            imn = np.where(dm16[..., None] == 0, 0, np.clip(_roundf(mins / dm16[..., None]), 0, smax)).astype(np.int32)
            dl = d16[..., None] * isc
            ml = dm16[..., None] * imn
            q = np.where(dl[..., None] == 0, 0, np.clip(_roundf((xs + ml[..., None]) / dl[..., None]), 0, qmax)).astype(np.int32)
        q = q.reshape(n, nblk, 256)
        if wt == Q2_K:
            out[..., 0:16] = (isc | (imn << 4)).astype(np.uint8)
            qs = np.zeros((n, nblk, 64), np.int32)
            for w in range(256):
                h, t, l = w // 128, (w // 32) % 4, w % 32
                qs[..., 32 * h + l] |= q[..., w] << (2 * t)
            out[..., 16:80] = qs.astype(np.uint8)
            out[..., 80:82] = _f16_bytes(d16)
            out[..., 82:84] = _f16_bytes(dm16)
        else:
            out[..., 0:2] = _f16_bytes(d16)
            out[..., 2:4] = _f16_bytes(dm16)
            s12 = np.zeros((n, nblk, 12), np.int32)
            for j in range(4):
                s12[..., j] = (isc[..., j] & 63) | ((isc[..., j + 4] >> 4) << 6)
                s12[..., j + 4] = (imn[..., j] & 63) | ((imn[..., j + 4] >> 4) << 6)
                s12[..., j + 8] = (isc[..., j + 4] & 0xF) | ((imn[..., j + 4] & 0xF) << 4)
            out[..., 4:16] = s12.astype(np.uint8)
            qs = np.zeros((n, nblk, 128), np.int32)
            qh = np.zeros((n, nblk, 32), np.int32)
            for w in range(256):
                ib, p = w // 32, w % 32
                qs[..., 32 * (ib >> 1) + p] |= (q[..., w] & 0xF) << (4 * (ib & 1))
                qh[..., p] |= ((q[..., w] >> 4) & 1) << ib
            if wt == Q4_K:
                out[..., 16:144] = qs.astype(np.uint8)
            else:
                out[..., 16:48] = qh.astype(np.uint8)
                out[..., 48:176] = qs.astype(np.uint8)
    elif wt in (Q3_K, Q6_K):
        qoff = 4 if wt == Q3_K else 32
        xs = x.reshape(n, nblk, 16, 16)
        imax = np.abs(xs).argmax(-1)
        mx = np.take_along_axis(xs, imax[..., None], -1)[..., 0]
        scale = mx / -qoff
        smax = 31 if wt == Q3_K else 127
        d = np.abs(scale).max(-1) / smax
        d16 = d.astype(np.float16).astype(np.float32)
        with np.errstate(divide="ignore", invalid="ignore"):
            isc = np.where(d16[..., None] == 0, 0, np.clip(_roundf(scale / d16[..., None]), -smax - 1, smax)).astype(np.int32)
            dl = d16[..., None] * isc
            q = np.where(dl[..., None] == 0, 0, np.clip(_roundf(xs / dl[..., None]), -qoff, qoff - 1)).astype(np.int32)
        u = (q + qoff).reshape(n, nblk, 256)
        if wt == Q3_K:
            hm = np.zeros((n, nblk, 32), np.int32)
            qs = np.zeros((n, nblk, 64), np.int32)
            for w in range(256):
                h, j, l = w // 128, (w // 32) % 4, w % 32
                qs[..., 32 * h + l] |= (u[..., w] & 3) << (2 * j)
                hm[..., l] |= ((u[..., w] >> 2) & 1) << (4 * h + j)
            us = isc + 32
            s12 = np.zeros((n, nblk, 12), np.int32)
            for i in range(16):
                s12[..., i % 8] |= (us[..., i] & 0xF) << (4 * (i // 8))
                s12[..., 8 + i % 4] |= ((us[..., i] >> 4) & 3) << (2 * (i // 4))
            out[..., 0:32] = hm.astype(np.uint8)
            out[..., 32:96] = qs.astype(np.uint8)
            out[..., 96:108] = s12.astype(np.uint8)
            out[..., 108:110] = _f16_bytes(d16)
        else:
            ql = np.zeros((n, nblk, 128), np.int32)
            qh = np.zeros((n, nblk, 64), np.int32)
            for w in range(256):
                h, t, p = w // 128, (w // 32) % 4, w % 32
                ql[..., 64 * h + 32 * (t & 1) + p] |= (u[..., w] & 0xF) << (4 * (t >> 1))
                qh[..., 32 * h + p] |= ((u[..., w] >> 4) & 3) << (2 * t)
            out[..., 0:128] = ql.astype(np.uint8)
            out[..., 128:192] = qh.astype(np.uint8)
            out[..., 192:208] = isc.astype(np.int8).view(np.uint8)
            out[..., 208:210] = _f16_bytes(d16)
    elif wt == IQ3_S:
        raise NotImplementedError("IQ3_S has no quantizer here (gguf-py has none either): use random_blocks")
    else:
        raise NotImplementedError(f"GGML type {wt}")
    return out.reshape(n, nblk * bb)


def make_weights(rng: np.random.Generator, n: int, K: int, wt: int, std: float = 0.02) -> np.ndarray:
    """BASELINE's synthetic weights: N(0, std) quantized to the type, or random valid blocks for
    the types without a quantizer (IQ3_S)."""
    if wt == IQ3_S:
        return random_blocks(rng, n, K, wt)
    return quantize(rng.normal(0.0, std, size=(n, K)).astype(np.float32), wt)


def matmul_ref(x: np.ndarray, Wf: np.ndarray) -> np.ndarray:
    """fp64 y = x @ W^T (the reference CPU path's matmul, in float64 for the tolerance check)."""
    return x.astype(np.float64) @ Wf.astype(np.float64).T


def rel_err(y: np.ndarray, ref: np.ndarray) -> float:
    """max |y - ref| over each output row's max |ref| (gguf-plugin/test_gluon_kq_gpu.py:81-86)."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if ref.size == 0:
        return 0.0
    scale = np.maximum(np.abs(ref).max(axis=1, keepdims=True), 1e-30)
    return float((np.abs(y - ref) / scale).max())
