"""Builds device blobs in the ncnn layouts the AWA entry points accept."""

from __future__ import annotations

import numpy as np

import awa_hip as A


def _host_dtype(elemsize: int):
    return np.float32 if elemsize == 4 else np.uint16


def _encode(x: np.ndarray, elemsize: int) -> np.ndarray:
    return np.ascontiguousarray(x, np.float32) if elemsize == 4 else A.f32_to_bf16_bits(x)


def _decode(x: np.ndarray, elemsize: int) -> np.ndarray:
    return x.astype(np.float32) if elemsize == 4 else A.bf16_bits_to_f32(x)


class DeviceMat:
    """A device buffer plus its ncnn descriptor."""

    def __init__(self, blob_kwargs: dict, total_elems: int, elemsize: int):
        self.buf = A.DeviceBuffer(max(total_elems, 1) * elemsize)
        self.elemsize = elemsize
        self.blob = A.mat(self.buf.ptr, elemsize=elemsize, **blob_kwargs)
        self.total = total_elems

    def upload_raw(self, host: np.ndarray) -> None:
        self.buf.upload(host)

    def download_raw(self) -> np.ndarray:
        return self.buf.download((self.total,), _host_dtype(self.elemsize))


def qkv_blob(qkv: np.ndarray, layout: str, elemsize: int) -> DeviceMat:
    """qkv [T][3][H][d] fp32 -> device blob in layout 'a' Mat(d,3H,T), 'b' Mat(d,H,3T),
    'c' NCNN_BATCH Mat(d,H,3; n=T) with 4 KiB batch padding, 'd' Mat(d,H,3,T)."""
    T, three, H, d = qkv.shape
    assert three == 3
    enc = _encode(qkv, elemsize)
    if layout == "a":
        m = DeviceMat(dict(w=d, h=3 * H, c=T, dims=3), T * 3 * H * d, elemsize)
        assert m.blob.cstep == 3 * H * d
        m.upload_raw(enc.reshape(-1))
    elif layout == "b":
        m = DeviceMat(dict(w=d, h=H, c=3 * T, dims=3), 3 * T * H * d, elemsize)
        m.upload_raw(np.ascontiguousarray(enc.transpose(1, 0, 2, 3)).reshape(-1))
    elif layout == "c":
        cstep = A.align_cstep(H * d, elemsize)
        nstep = (3 * cstep * elemsize + 4095) // 4096 * 4096 // elemsize
        m = DeviceMat(dict(w=d, h=H, c=3, dims=3, n=T, cstep=cstep, nstep=nstep), T * nstep, elemsize)
        host = np.zeros((T, nstep), enc.dtype)
        host[:, : 3 * H * d] = enc.reshape(T, -1)
        m.upload_raw(host.reshape(-1))
    elif layout == "d":
        m = DeviceMat(dict(w=d, h=H, d=3, c=T, dims=4), T * 3 * H * d, elemsize)
        m.upload_raw(enc.reshape(-1))
    else:
        raise ValueError(layout)
    return m


def video_out_blob(t: int, h: int, w: int, heads: int, d: int, elemsize: int, batch: bool) -> DeviceMat:
    """Video output: Mat(d, H, N) or NCNN_BATCH Mat(d, H, w, h; n = t) with 4 KiB batch padding."""
    if not batch:
        return DeviceMat(dict(w=d, h=heads, c=t * h * w, dims=3), t * h * w * heads * d, elemsize)
    cstep = A.align_cstep(d * heads * w, elemsize)
    nstep = (h * cstep * elemsize + 4095) // 4096 * 4096 // elemsize
    return DeviceMat(dict(w=d, h=heads, d=w, c=h, dims=4, n=t, cstep=cstep, nstep=nstep), t * nstep, elemsize)


def read_video(m: DeviceMat, t: int, h: int, w: int, heads: int, d: int) -> np.ndarray:
    raw = _decode(m.download_raw(), m.elemsize)
    if m.blob.dims == 3:
        return raw[: t * h * w * heads * d].reshape(t * h * w, heads, d)
    out = np.zeros((t, h, w, heads, d), np.float32)
    for ti in range(t):
        for hi in range(h):
            base = ti * m.blob.nstep + hi * m.blob.cstep
            out[ti, hi] = raw[base: base + w * heads * d].reshape(w, heads, d)
    return out.reshape(t * h * w, heads, d)


def mat3(w: int, h: int, c: int, elemsize: int) -> DeviceMat:
    return DeviceMat(dict(w=w, h=h, c=c, dims=3), c * A.align_cstep(w * h, elemsize), elemsize)


def read_mat3(m: DeviceMat) -> np.ndarray:
    raw = _decode(m.download_raw(), m.elemsize)
    b = m.blob
    return raw.reshape(b.c, b.cstep)[:, : b.w * b.h].reshape(b.c, b.h, b.w)


def upload_mat3(m: DeviceMat, x: np.ndarray) -> None:
    b = m.blob
    host = np.zeros((b.c, b.cstep), _host_dtype(m.elemsize))
    host[:, : b.w * b.h] = _encode(x, m.elemsize).reshape(b.c, -1)
    m.upload_raw(host.reshape(-1))
