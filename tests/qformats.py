"""Independent numpy decoders of the GGUF block formats, for the tests.

Written from the published ggml block layouts (ggml-common.h block_q8_0,
block_q5_0, block_q4_K, block_q6_K) as whole-array numpy operations, so they
share no code with the oracle's C decoders: a wrong nibble order, scale
packing or sign in either one makes the two disagree.
"""
import numpy as np

F32, F16, Q5_0, Q8_0, Q4_K, Q6_K = 0, 1, 6, 8, 12, 14
BLOCK = {F32: (1, 4), F16: (1, 2), Q5_0: (32, 22), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}


def _f16(b, off):
    return b[:, off:off + 2].copy().view(np.float16).astype(np.float32)[:, 0]


def decode(typ, raw, n):
    """Rows of `raw` (bytes) -> float32 [rows, n]."""
    be, bb = BLOCK[typ]
    raw = np.ascontiguousarray(raw, np.uint8)
    if typ == F32:
        return raw.view(np.float32).reshape(-1, n).copy()
    if typ == F16:
        return raw.view(np.float16).astype(np.float32).reshape(-1, n)
    b = raw.reshape(-1, bb)  # one row per block
    if typ == Q8_0:
        d = _f16(b, 0)
        q = b[:, 2:34].view(np.int8).astype(np.float32)
        y = d[:, None] * q
    elif typ == Q5_0:
        d = _f16(b, 0)
        qh = b[:, 2:6].copy().view(np.uint32)[:, 0]
        qs = b[:, 6:22]
        j = np.arange(16)
        lo = (qs & 0xF) | (((qh[:, None] >> j) & 1) << 4).astype(np.uint8)
        hi = (qs >> 4) | (((qh[:, None] >> (j + 16)) & 1) << 4).astype(np.uint8)
        q = np.concatenate([lo, hi], axis=1).astype(np.float32) - 16.0
        y = d[:, None] * q
    elif typ == Q4_K:
        d, dmin = _f16(b, 0), _f16(b, 2)
        s = b[:, 4:16].astype(np.int32)
        sc = np.empty((b.shape[0], 8), np.int32)
        mn = np.empty((b.shape[0], 8), np.int32)
        sc[:, :4] = s[:, 0:4] & 63
        mn[:, :4] = s[:, 4:8] & 63
        sc[:, 4:] = (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)
        mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
        qs = b[:, 16:144].reshape(-1, 4, 32)
        q = np.empty((b.shape[0], 8, 32), np.float32)
        q[:, 0::2, :] = qs & 0xF   # sub-block 2c: low nibbles of chunk c
        q[:, 1::2, :] = qs >> 4    # sub-block 2c+1: high nibbles
        d1 = (d[:, None] * sc.astype(np.float32)).astype(np.float32)
        m1 = (dmin[:, None] * mn.astype(np.float32)).astype(np.float32)
        y = (d1[:, :, None] * q - m1[:, :, None]).reshape(-1, 256)
    elif typ == Q6_K:
        ql = b[:, 0:128].astype(np.int32).reshape(-1, 2, 64)
        qh = b[:, 128:192].astype(np.int32).reshape(-1, 2, 32)
        sc = b[:, 192:208].view(np.int8).astype(np.float32).reshape(-1, 2, 8)
        d = _f16(b, 208)
        q = np.empty((b.shape[0], 2, 4, 32), np.int32)
        q[:, :, 0] = (ql[:, :, 0:32] & 0xF) | (((qh >> 0) & 3) << 4)
        q[:, :, 1] = (ql[:, :, 32:64] & 0xF) | (((qh >> 2) & 3) << 4)
        q[:, :, 2] = (ql[:, :, 0:32] >> 4) | (((qh >> 4) & 3) << 4)
        q[:, :, 3] = (ql[:, :, 32:64] >> 4) | (((qh >> 6) & 3) << 4)
        q = (q - 32).astype(np.float32)
        # element l of quarter g (l in 0..31) uses scale sc[2*g + l // 16]
        scale = np.stack([sc[:, :, 2 * g:2 * g + 2].repeat(16, axis=2) for g in range(4)], axis=2)
        y = ((d[:, None, None, None] * scale).astype(np.float32) * q).reshape(-1, 256)
    else:
        raise ValueError(typ)
    return y.astype(np.float32).reshape(-1, n)


def encode_q8_0(v):
    """A simple Q8_0 encoder (round-to-nearest, d = amax/127) for building
    hand-made weights in tests."""
    v = np.asarray(v, np.float32).reshape(-1, 32)
    amax = np.abs(v).max(axis=1)
    d = (amax / 127.0).astype(np.float16)
    df = d.astype(np.float32)
    q = np.where(df[:, None] > 0, np.rint(v / np.where(df > 0, df, 1)[:, None]), 0).clip(-127, 127).astype(np.int8)
    out = np.empty((v.shape[0], 34), np.uint8)
    out[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(-1)
