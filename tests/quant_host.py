"""Host restatement of ggml's block formats and integer dot products (ggml
@ e6f2ec01f, the version the reference's fixtures were made with: ggml-common.h
layouts, ggml-quants.c dequantize_row_* / quantize_row_*_ref, ggml-cpu's
generic vec_dot_*), as the reference restates them (S/quant/*.hpp,
S/kernels/dot.hpp). Test infrastructure: the checker for the device
kernels, pinned here against the reference's quant_golden.gguf and
kernel_golden.gguf."""
from __future__ import annotations

import numpy as np

from synapse_amd.gguf import BF16, BLOCK, F16, F32, Q4_0, Q4_K, Q5_0, Q6_K, Q8_0, Q8_K

f32 = np.float32


def _h(b: np.ndarray) -> np.ndarray:
    """Little-endian binary16 from byte pairs [..., 2] -> float32."""
    return b.copy().view(np.float16).astype(f32).reshape(b.shape[:-1])


def blocks(raw: np.ndarray, t: int) -> np.ndarray:
    bs, ts = BLOCK[t]
    return raw.reshape(-1, ts)


def dequantize(raw: np.ndarray, t: int) -> np.ndarray:
    """Every element of a tensor's bytes, in order, as float32."""
    if t == F32:
        return raw.view(f32).copy()
    if t == F16:
        return raw.view(np.float16).astype(f32)
    if t == BF16:
        return (raw.view(np.uint16).astype(np.uint32) << 16).view(f32)
    b = blocks(raw, t)
    if t == Q4_0:
        d = _h(b[:, 0:2])[:, None]
        qs = b[:, 2:18].astype(np.int32)
        lo, hi = (qs & 0xF) - 8, (qs >> 4) - 8
        return (np.concatenate([lo, hi], 1).astype(f32) * d).reshape(-1)
    if t == Q5_0:
        d = _h(b[:, 0:2])[:, None]
        qh = b[:, 2:6].copy().view(np.uint32).astype(np.int64)  # [n, 1]
        qs = b[:, 6:22].astype(np.int64)
        j = np.arange(16)
        xh0 = ((qh >> j) << 4) & 0x10
        xh1 = (qh >> (j + 12)) & 0x10
        lo = ((qs & 0xF) | xh0) - 16
        hi = ((qs >> 4) | xh1) - 16
        return (np.concatenate([lo, hi], 1).astype(f32) * d).reshape(-1)
    if t == Q8_0:
        d = _h(b[:, 0:2])[:, None]
        return (b[:, 2:34].view(np.int8).astype(f32) * d).reshape(-1)
    if t == Q4_K:
        out = np.empty((b.shape[0], 256), f32)
        d, dmin = _h(b[:, 0:2]), _h(b[:, 2:4])
        sc12 = b[:, 4:16].astype(np.int32)
        qs = b[:, 16:144].astype(np.int32)
        for i in range(b.shape[0]):
            for g in range(4):
                q = qs[i, 32 * g:32 * g + 32]
                for half in range(2):
                    sc, m = scale_min_k4(2 * g + half, sc12[i])
                    dd, mm = d[i] * f32(sc), dmin[i] * f32(m)
                    v = (q & 0xF) if half == 0 else (q >> 4)
                    out[i, 64 * g + 32 * half:64 * g + 32 * half + 32] = dd * v.astype(f32) - mm
        return out.reshape(-1)
    if t == Q6_K:
        out = np.empty((b.shape[0], 256), f32)
        ql = b[:, 0:128].astype(np.int32)
        qh = b[:, 128:192].astype(np.int32)
        sc = b[:, 192:208].view(np.int8).astype(np.int32)
        d = _h(b[:, 208:210])
        for i in range(b.shape[0]):
            for n in range(2):
                l = np.arange(32)
                QL, QH, S = ql[i, 64 * n:], qh[i, 32 * n:], sc[i, 8 * n:]
                q1 = ((QL[l] & 0xF) | (((QH[l] >> 0) & 3) << 4)) - 32
                q2 = ((QL[l + 32] & 0xF) | (((QH[l] >> 2) & 3) << 4)) - 32
                q3 = ((QL[l] >> 4) | (((QH[l] >> 4) & 3) << 4)) - 32
                q4 = ((QL[l + 32] >> 4) | (((QH[l] >> 6) & 3) << 4)) - 32
                isx = l // 16
                base = 128 * n
                for k, q in enumerate((q1, q2, q3, q4)):
                    out[i, base + 32 * k + l] = (d[i] * S[isx + 2 * k].astype(f32)) * q.astype(f32)
        return out.reshape(-1)
    raise ValueError(f"type {t}")


def scale_min_k4(j: int, q: np.ndarray) -> tuple[int, int]:
    """The 6-bit (scale, min) of sub-block j of a Q4_K super-block."""
    if j < 4:
        return int(q[j] & 63), int(q[j + 4] & 63)
    return int((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4)), int((q[j + 4] >> 4) | ((q[j] >> 6) << 4))


# ---- activation quantizers (ggml's reference quantizers) ---------------------

def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    """quantize_row_q8_0_ref: per 32, d = amax / 127 (stored binary16),
    q = round-half-away(x / d)."""
    x = np.asarray(x, f32).reshape(-1, 32)
    out = np.zeros((x.shape[0], 34), np.uint8)
    for i, row in enumerate(x):
        amax = f32(np.max(np.abs(row)))
        d = f32(amax / f32(127))
        idv = f32(1) / d if d != 0 else f32(0)
        v = row * idv
        t = np.trunc(v)  # roundf: half away from zero, decided on the exact fraction
        q = t + np.where(np.abs(v - t) >= f32(0.5), np.sign(v), f32(0))
        out[i, 0:2] = np.array([d], np.float16).view(np.uint8)
        out[i, 2:34] = q.astype(np.int8).view(np.uint8)
    return out.reshape(-1)


def _nearest_int(v: np.ndarray) -> np.ndarray:
    """Round half to even through the 1.5 * 2^23 trick (float add)."""
    t = (v.astype(f32) + f32(12582912.0)).view(np.int32)
    return (t & 0x007FFFFF) - 0x00400000


def quantize_q8_k(x: np.ndarray) -> np.ndarray:
    """quantize_row_q8_K_ref: per 256, the signed value of largest magnitude
    max, iscale = -127 / max, q = min(127, nearest_int(iscale x)),
    d = 1 / iscale, and the 16 sums of 16."""
    x = np.asarray(x, f32).reshape(-1, 256)
    out = np.zeros((x.shape[0], 292), np.uint8)
    for i, row in enumerate(x):
        amax, mx = f32(0), f32(0)
        for v in row:
            if abs(v) > amax:
                amax, mx = f32(abs(v)), v
        if amax == 0:
            continue  # d = 0, q = 0, sums 0
        iscale = f32(-127) / mx
        q = np.minimum(127, _nearest_int(iscale * row)).astype(np.int8)
        out[i, 0:4] = np.array([f32(1) / iscale], f32).view(np.uint8)
        out[i, 4:260] = q.view(np.uint8)
        out[i, 260:292] = q.astype(np.int32).reshape(16, 16).sum(1).astype(np.int16).view(np.uint8)
    return out.reshape(-1)


def act_type(t: int) -> int:
    """The activation format ggml pairs with a weight format (vec_dot_type)."""
    return Q8_K if t in (Q4_K, Q6_K) else Q8_0


def quantize_act(x: np.ndarray, t: int) -> np.ndarray:
    return quantize_q8_k(x) if act_type(t) == Q8_K else quantize_q8_0(x)


# ---- integer dot products ------------------------------------------------------

def vec_dot(w_row: np.ndarray, t: int, act: np.ndarray) -> float:
    """One weight row (t blocks) against quantized activations: per block an
    exact integer sum, combined in float with the block scales."""
    if t in (F32, F16, BF16):
        return float(np.dot(dequantize(w_row, t).astype(np.float64), act.astype(np.float64)))
    wb = blocks(w_row, t)
    if act_type(t) == Q8_0:
        ab = blocks(act, Q8_0)
        dy = _h(ab[:, 0:2])
        qy = ab[:, 2:34].view(np.int8).astype(np.int64)
        dx = _h(wb[:, 0:2])
        if t == Q8_0:
            qx = wb[:, 2:34].view(np.int8).astype(np.int64)
        elif t == Q4_0:
            qs = wb[:, 2:18].astype(np.int64)
            qx = np.concatenate([(qs & 0xF) - 8, (qs >> 4) - 8], 1)
        elif t == Q5_0:
            qh = wb[:, 2:6].copy().view(np.uint32).astype(np.int64)
            qs = wb[:, 6:22].astype(np.int64)
            j = np.arange(16)
            qx = np.concatenate([((qs & 0xF) | (((qh >> j) << 4) & 0x10)) - 16,
                                 ((qs >> 4) | ((qh >> (j + 12)) & 0x10)) - 16], 1)
        s = f32(0)
        for i in range(wb.shape[0]):
            sumi = int(np.sum(qx[i] * qy[i]))
            s = f32(s + f32(sumi) * (dx[i] * dy[i]))
        return float(s)
    ab = blocks(act, Q8_K)
    s = f32(0)
    for i in range(wb.shape[0]):
        yd = ab[i, 0:4].copy().view(f32)[0]
        qy = ab[i, 4:260].view(np.int8).astype(np.int64)
        bsums = ab[i, 260:292].copy().view(np.int16).astype(np.int64)
        if t == Q4_K:
            d, dmin = _h(wb[i, 0:2])[()], _h(wb[i, 2:4])[()]
            sc12 = wb[i, 4:16].astype(np.int32)
            qs = wb[i, 16:144].astype(np.int64)
            acc, accm = 0, 0
            for g in range(4):
                for half in range(2):
                    sc, m = scale_min_k4(2 * g + half, sc12)
                    q = (qs[32 * g:32 * g + 32] & 0xF) if half == 0 else (qs[32 * g:32 * g + 32] >> 4)
                    sub = 2 * g + half
                    acc += sc * int(np.sum(q * qy[32 * sub:32 * sub + 32]))
                    accm += m * int(bsums[2 * sub] + bsums[2 * sub + 1])
            s = f32(s + f32(d * yd) * f32(acc) - f32(dmin * yd) * f32(accm))
        elif t == Q6_K:
            d = _h(wb[i, 208:210])[()]
            ql = wb[i, 0:128].astype(np.int64)
            qh = wb[i, 128:192].astype(np.int64)
            sc = wb[i, 192:208].view(np.int8).astype(np.int64)
            acc = 0
            for n in range(2):
                l = np.arange(32)
                QL, QH = ql[64 * n:], qh[32 * n:]
                qq = [((QL[l] & 0xF) | (((QH[l] >> 0) & 3) << 4)) - 32, ((QL[l + 32] & 0xF) | (((QH[l] >> 2) & 3) << 4)) - 32,
                      ((QL[l] >> 4) | (((QH[l] >> 4) & 3) << 4)) - 32, ((QL[l + 32] >> 4) | (((QH[l] >> 6) & 3) << 4)) - 32]
                for k in range(4):
                    for h16 in range(2):
                        idx = 128 * n + 32 * k + 16 * h16
                        acc += int(sc[8 * n + 2 * k + h16]) * int(np.sum(qq[k][16 * h16:16 * h16 + 16] * qy[idx:idx + 16]))
            s = f32(s + f32(d * yd) * f32(acc))
        else:
            raise ValueError(f"type {t}")
    return float(s)


def dequantize_act(act: np.ndarray, t: int) -> np.ndarray:
    """x^ = d q of quantized activations (what the integer dot sees)."""
    if t == Q8_0:
        b = blocks(act, Q8_0)
        return (b[:, 2:34].view(np.int8).astype(f32) * _h(b[:, 0:2])[:, None]).reshape(-1)
    b = blocks(act, Q8_K)
    return (b[:, 4:260].view(np.int8).astype(f32) * b[:, 0:4].copy().view(f32)).reshape(-1)
