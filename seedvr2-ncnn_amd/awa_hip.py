"""Python (ctypes) binding of libseedvr2_awa.so, the C ABI declared in
include/seedvr2_awa.h.

This is the Python-side mirror a ctypes caller (for example the reference's
Python tooling) would use. It exposes plans, device buffers, streams/events
and the forward entry points; it never computes anything itself. The library
is loaded from this directory and the import fails loudly when it is missing.
"""

from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libseedvr2_awa.so")

AWA_OK = 0
AWA_ERR_INVALID = -1
AWA_ERR_DEVICE = -2
AWA_ERR_ALLOC = -100
COMPUTE_F32 = 0  # exact-score fp32 kernel (int8 digit slices + bf16 pieces)
COMPUTE_BF16 = 1
COMPUTE_F32_MFMA = 2  # fp32 MFMA with plain accumulation (comparison path)

# Every symbol of include/seedvr2_awa.h.
EXPORTED_SYMBOLS = (
    "awa_last_error", "awa_device_count", "awa_runtime_init", "awa_malloc", "awa_free", "awa_host_alloc",
    "awa_host_free", "awa_memcpy_h2d", "awa_memcpy_d2h", "awa_memcpy_d2d", "awa_zero", "awa_stream_create",
    "awa_stream_destroy", "awa_stream_synchronize", "awa_event_create", "awa_event_destroy", "awa_event_record",
    "awa_event_synchronize", "awa_event_elapsed_ms", "awa_fill_normal", "awa_fill_normal_scaled", "awa_plan_create", "awa_plan_destroy",
    "awa_plan_info_get", "awa_plan_windows", "awa_plan_sequence_index", "awa_plan_cu_seqlens",
    "awa_plan_video_positions", "awa_plan_text_positions", "awa_plan_rope_table", "awa_plan_upload",
    "awa_plan_attention_split",
    "awa_qkv_shape", "awa_forward", "awa_forward_noalloc", "awa_forward_qknorm", "awa_rmsnorm", "awa_qkv_concat", "awa_pack", "awa_mmrope",
    "awa_window_attention", "awa_unpack", "awa_cast",
    "awa_stack_create", "awa_stack_destroy", "awa_stack_run", "awa_stack_set_profiling", "awa_stack_set_graph", "awa_stack_block_times",
    "awa_stack_block_flops", "awa_dit_block_create", "awa_dit_block_destroy", "awa_dit_block_forward",
    "awa_dit_stack_create", "awa_dit_stack_destroy", "awa_dit_stack_run", "awa_dit_stack_set_profiling",
    "awa_dit_stack_block_times",
)


class AwaQkNorm(ctypes.Structure):
    """awa_qk_norm: device gamma pointers (q video, k video, q text, k text), eps."""
    _fields_ = [
        ("q_video", ctypes.c_void_p),
        ("k_video", ctypes.c_void_p),
        ("q_text", ctypes.c_void_p),
        ("k_text", ctypes.c_void_p),
        ("eps", ctypes.c_float),
    ]


class AwaBlob(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dims", ctypes.c_int),
        ("w", ctypes.c_int),
        ("h", ctypes.c_int),
        ("d", ctypes.c_int),
        ("c", ctypes.c_int),
        ("n", ctypes.c_int),
        ("elemsize", ctypes.c_int),
        ("cstep", ctypes.c_longlong),
        ("nstep", ctypes.c_longlong),
    ]


class AwaPlanDesc(ctypes.Structure):
    _fields_ = [(name, ctypes.c_int) for name in (
        "source_t", "source_h", "source_w", "windows_t", "windows_h", "windows_w", "text_tokens", "shifted",
        "rope_dim", "runtime_t", "runtime_h", "runtime_w", "runtime_tokens", "heads")]


class AwaStackDesc(ctypes.Structure):
    _fields_ = [(name, ctypes.c_int) for name in (
        "source_t", "source_h", "source_w", "windows_t", "windows_h", "windows_w", "text_tokens", "blocks",
        "fp32_prefix_blocks", "heads", "head_dim")]


class AwaDitBlockDesc(ctypes.Structure):
    """awa_dit_block_desc."""
    _fields_ = [(name, ctypes.c_int) for name in (
        "source_t", "source_h", "source_w", "windows_t", "windows_h", "windows_w", "text_tokens", "shifted",
        "heads", "head_dim", "hidden", "mlp_hidden", "last_layer", "precision")] + [("norm_eps", ctypes.c_float)]


class AwaDitStackDesc(ctypes.Structure):
    """awa_dit_stack_desc."""
    _fields_ = [(name, ctypes.c_int) for name in (
        "source_t", "source_h", "source_w", "windows_t", "windows_h", "windows_w", "text_tokens", "blocks",
        "fp32_prefix_blocks", "heads", "head_dim", "hidden", "mlp_hidden")] + [("norm_eps", ctypes.c_float)]


class AwaDitBranchWeights(ctypes.Structure):
    """awa_dit_branch_weights: device pointers of one branch's weights."""
    _fields_ = [(name, ctypes.c_void_p) for name in (
        "qkv", "proj_out", "proj_out_bias", "mlp_gate", "mlp_in", "mlp_out", "norm_q", "norm_k", "ada")]


class AwaPlanInfo(ctypes.Structure):
    _fields_ = [(name, ctypes.c_int) for name in (
        "source_t", "source_h", "source_w", "source_tokens", "text_tokens", "window_count", "sequence_tokens",
        "window_t", "window_h", "window_w", "max_window_tokens", "rope_dim", "shifted")]


_LIB: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `make -C seedvr2-ncnn_amd`")
        L = ctypes.CDLL(LIB_PATH)
        vp, i, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
        L.awa_last_error.restype = ctypes.c_char_p
        L.awa_device_count.argtypes = [ctypes.POINTER(i)]
        L.awa_runtime_init.argtypes = [i]
        L.awa_malloc.argtypes = [ctypes.POINTER(vp), sz]
        L.awa_free.argtypes = [vp]
        L.awa_host_alloc.argtypes = [ctypes.POINTER(vp), sz]
        L.awa_host_free.argtypes = [vp]
        for name in ("awa_memcpy_h2d", "awa_memcpy_d2h", "awa_memcpy_d2d"):
            getattr(L, name).argtypes = [vp, vp, sz, vp]
        L.awa_zero.argtypes = [vp, sz, vp]
        L.awa_stream_create.argtypes = [ctypes.POINTER(vp)]
        L.awa_stream_destroy.argtypes = [vp]
        L.awa_stream_synchronize.argtypes = [vp]
        L.awa_event_create.argtypes = [ctypes.POINTER(vp)]
        L.awa_event_destroy.argtypes = [vp]
        L.awa_event_record.argtypes = [vp, vp]
        L.awa_event_synchronize.argtypes = [vp]
        L.awa_event_elapsed_ms.argtypes = [vp, vp, ctypes.POINTER(ctypes.c_float)]
        L.awa_fill_normal.argtypes = [vp, sz, i, ctypes.c_ulonglong, vp]
        L.awa_fill_normal_scaled.argtypes = [vp, sz, i, ctypes.c_ulonglong, ctypes.c_float, vp]
        L.awa_plan_create.argtypes = [ctypes.POINTER(AwaPlanDesc), ctypes.POINTER(vp)]
        L.awa_plan_destroy.argtypes = [vp]
        L.awa_plan_destroy.restype = None
        L.awa_plan_info_get.argtypes = [vp, ctypes.POINTER(AwaPlanInfo)]
        for name in ("awa_plan_windows", "awa_plan_sequence_index", "awa_plan_cu_seqlens",
                     "awa_plan_video_positions", "awa_plan_text_positions"):
            getattr(L, name).argtypes = [vp, vp]
        L.awa_plan_rope_table.argtypes = [vp, vp]
        L.awa_plan_upload.argtypes = [vp, vp]
        L.awa_plan_attention_split.argtypes = [vp, i, i, ctypes.POINTER(i)]
        bp = ctypes.POINTER(AwaBlob)
        L.awa_forward.argtypes = [vp, bp, bp, bp, bp, i, vp]
        L.awa_forward_noalloc.argtypes = [vp, bp, bp, bp, bp, i, vp]
        L.awa_forward_qknorm.argtypes = [vp, bp, bp, ctypes.POINTER(AwaQkNorm), bp, bp, i, vp]
        L.awa_rmsnorm.argtypes = [bp, vp, ctypes.c_float, bp, vp]
        L.awa_qkv_concat.argtypes = [bp, bp, bp, bp, vp]
        L.awa_pack.argtypes = [vp, bp, bp, bp, bp, vp]
        L.awa_mmrope.argtypes = [vp, bp, bp, vp]
        L.awa_window_attention.argtypes = [vp, bp, bp, i, vp]
        L.awa_unpack.argtypes = [vp, bp, bp, bp, vp]
        L.awa_cast.argtypes = [bp, bp, vp]
        L.awa_stack_create.argtypes = [ctypes.POINTER(AwaStackDesc), ctypes.POINTER(vp)]
        L.awa_stack_destroy.argtypes = [vp]
        L.awa_stack_destroy.restype = None
        vpp = ctypes.POINTER(vp)
        L.awa_stack_run.argtypes = [vp, vpp, vpp, vpp, vpp, vp]
        L.awa_stack_set_profiling.argtypes = [vp, i]
        L.awa_stack_block_times.argtypes = [vp, ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_float)]
        L.awa_stack_block_flops.argtypes = [vp, ctypes.POINTER(ctypes.c_double)]
        L.awa_dit_block_create.argtypes = [ctypes.POINTER(AwaDitBlockDesc), ctypes.POINTER(vp)]
        L.awa_dit_block_destroy.argtypes = [vp]
        L.awa_dit_block_destroy.restype = None
        wp = ctypes.POINTER(AwaDitBranchWeights)
        L.awa_dit_block_forward.argtypes = [vp, wp, wp, vp, vp, vp, vp, vp, vp]
        L.awa_dit_stack_create.argtypes = [ctypes.POINTER(AwaDitStackDesc), ctypes.POINTER(vp)]
        L.awa_dit_stack_destroy.argtypes = [vp]
        L.awa_dit_stack_destroy.restype = None
        L.awa_dit_stack_run.argtypes = [vp, wp, wp, vp, vp, vp, vp, vp, vp]
        L.awa_dit_stack_set_profiling.argtypes = [vp, i]
        L.awa_dit_stack_block_times.argtypes = [vp, ctypes.POINTER(ctypes.c_float)]
        _LIB = L
    return _LIB


class AwaError(RuntimeError):
    def __init__(self, code: int, where: str):
        msg = lib().awa_last_error().decode(errors="replace")
        super().__init__(f"{where} failed with {code}: {msg}")
        self.code = code


def check(code: int, where: str) -> None:
    if code != AWA_OK:
        raise AwaError(code, where)


def device_count() -> int:
    n = ctypes.c_int(0)
    check(lib().awa_device_count(ctypes.byref(n)), "awa_device_count")
    return n.value


def init(device: int = 0) -> None:
    check(lib().awa_runtime_init(device), "awa_runtime_init")


# ---- device memory ----

class DeviceBuffer:
    """Owned device allocation."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(lib().awa_malloc(ctypes.byref(p), self.nbytes), "awa_malloc")
        self.ptr = p.value or 0

    def free(self) -> None:
        if self.ptr:
            lib().awa_free(ctypes.c_void_p(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def upload(self, array: np.ndarray, stream: Optional["Stream"] = None) -> None:
        a = np.ascontiguousarray(array)
        assert a.nbytes <= self.nbytes
        check(lib().awa_memcpy_h2d(ctypes.c_void_p(self.ptr), a.ctypes.data_as(ctypes.c_void_p), a.nbytes,
                                   _s(stream)), "awa_memcpy_h2d")
        synchronize(stream)

    def download(self, shape, dtype, stream: Optional["Stream"] = None) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        check(lib().awa_memcpy_d2h(out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(self.ptr), out.nbytes,
                                   _s(stream)), "awa_memcpy_d2h")
        synchronize(stream)
        return out

    def zero(self, stream: Optional["Stream"] = None) -> None:
        check(lib().awa_zero(ctypes.c_void_p(self.ptr), self.nbytes, _s(stream)), "awa_zero")

    def fill_normal(self, count: int, elemsize: int, seed: int, stream: Optional["Stream"] = None,
                    stddev: float = 1.0) -> None:
        check(lib().awa_fill_normal_scaled(ctypes.c_void_p(self.ptr), count, elemsize, seed, stddev, _s(stream)),
              "awa_fill_normal_scaled")


class Stream:
    def __init__(self):
        p = ctypes.c_void_p()
        check(lib().awa_stream_create(ctypes.byref(p)), "awa_stream_create")
        self.handle = p.value

    def synchronize(self) -> None:
        check(lib().awa_stream_synchronize(ctypes.c_void_p(self.handle)), "awa_stream_synchronize")

    def destroy(self) -> None:
        if self.handle:
            lib().awa_stream_destroy(ctypes.c_void_p(self.handle))
            self.handle = None


class Event:
    def __init__(self):
        p = ctypes.c_void_p()
        check(lib().awa_event_create(ctypes.byref(p)), "awa_event_create")
        self.handle = p.value

    def record(self, stream: Optional[Stream] = None) -> None:
        check(lib().awa_event_record(ctypes.c_void_p(self.handle), _s(stream)), "awa_event_record")

    def synchronize(self) -> None:
        check(lib().awa_event_synchronize(ctypes.c_void_p(self.handle)), "awa_event_synchronize")

    def elapsed_ms(self, stop: "Event") -> float:
        ms = ctypes.c_float()
        check(lib().awa_event_elapsed_ms(ctypes.c_void_p(self.handle), ctypes.c_void_p(stop.handle),
                                         ctypes.byref(ms)), "awa_event_elapsed_ms")
        return float(ms.value)

    def destroy(self) -> None:
        if self.handle:
            lib().awa_event_destroy(ctypes.c_void_p(self.handle))
            self.handle = None


def _s(stream: Optional[Stream]) -> ctypes.c_void_p:
    return ctypes.c_void_p(stream.handle if stream is not None else None)


def synchronize(stream: Optional[Stream] = None) -> None:
    check(lib().awa_stream_synchronize(_s(stream)), "awa_stream_synchronize")


# ---- blob descriptors (ncnn Mat semantics) ----

def align_cstep(elems: int, elemsize: int) -> int:
    """ncnn's cstep: channel size rounded up to 16 bytes, in elements."""
    return ((elems * elemsize + 15) // 16 * 16) // elemsize


def mat(ptr: int, w: int, h: int = 1, c: int = 1, elemsize: int = 4, d: int = 1, dims: Optional[int] = None,
        n: int = 1, cstep: Optional[int] = None, nstep: Optional[int] = None) -> AwaBlob:
    if dims is None:
        dims = 4 if d > 1 else (3 if c > 1 else (2 if h > 1 else 1))
    plane = w * (h if dims >= 2 else 1) * (d if dims == 4 else 1)
    cs = cstep if cstep is not None else (align_cstep(plane, elemsize) if dims >= 3 else plane)
    ns = nstep if nstep is not None else cs * (c if dims >= 3 else 1)
    return AwaBlob(ptr, dims, w, h, d, c, n, elemsize, cs, ns)


# ---- plans ----

@dataclass(frozen=True)
class LayerParams:
    """The reference layer's params 0-8 (src/awa/awa_layers.cpp:90-114, :872)."""

    t: int
    h: int
    w: int
    nt: int
    nh: int
    nw: int
    text_tokens: int
    shifted: bool = False
    rope_dim: int = 126


class Plan:
    def __init__(self, params: LayerParams, runtime: Optional[Sequence[int]] = None, heads: int = 0):
        """heads > 0: awa_plan_upload also builds the work list for that head
        count (what forward_noalloc needs)."""
        desc = AwaPlanDesc(params.t, params.h, params.w, params.nt, params.nh, params.nw, params.text_tokens,
                           int(params.shifted), params.rope_dim, 0, 0, 0, 0, heads)
        if runtime is not None:
            desc.runtime_t, desc.runtime_h, desc.runtime_w, desc.runtime_tokens = runtime
        p = ctypes.c_void_p()
        check(lib().awa_plan_create(ctypes.byref(desc), ctypes.byref(p)), "awa_plan_create")
        self.handle = p.value
        info = AwaPlanInfo()
        check(lib().awa_plan_info_get(ctypes.c_void_p(self.handle), ctypes.byref(info)), "awa_plan_info_get")
        self.info = info

    def destroy(self) -> None:
        if self.handle:
            lib().awa_plan_destroy(ctypes.c_void_p(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass

    @property
    def h(self) -> ctypes.c_void_p:
        return ctypes.c_void_p(self.handle)

    def _table(self, fn, count, dtype=np.int32, shape=None):
        out = np.zeros(count if shape is None else shape, dtype)
        check(fn(self.h, out.ctypes.data_as(ctypes.c_void_p)), fn.__name__)
        return out

    def windows(self) -> np.ndarray:
        return self._table(lib().awa_plan_windows, None, shape=(self.info.window_count, 6))

    def sequence_index(self) -> np.ndarray:
        return self._table(lib().awa_plan_sequence_index, self.info.sequence_tokens)

    def cu_seqlens(self) -> np.ndarray:
        return self._table(lib().awa_plan_cu_seqlens, self.info.window_count + 1)

    def video_positions(self) -> np.ndarray:
        return self._table(lib().awa_plan_video_positions, self.info.source_tokens)

    def text_positions(self) -> np.ndarray:
        return self._table(lib().awa_plan_text_positions, self.info.window_count * self.info.text_tokens)

    def rope_table(self) -> np.ndarray:
        return self._table(lib().awa_plan_rope_table, None, np.float32,
                           shape=(self.info.sequence_tokens, 2 * self.info.rope_dim))

    def upload(self, stream: Optional[Stream] = None) -> None:
        check(lib().awa_plan_upload(self.h, _s(stream)), "awa_plan_upload")

    def attention_split(self, heads: int, compute: int) -> int:
        """Key segments per (window, head) unit of this layer (1: not split)."""
        s = ctypes.c_int()
        check(lib().awa_plan_attention_split(self.h, heads, compute, ctypes.byref(s)), "awa_plan_attention_split")
        return s.value

    # forward entry points (blobs are AwaBlob descriptors of device memory)
    def forward(self, video_qkv: AwaBlob, text_qkv: AwaBlob, video_out: AwaBlob, text_out: AwaBlob,
                compute: int, stream: Optional[Stream] = None) -> None:
        check(lib().awa_forward(self.h, ctypes.byref(video_qkv), ctypes.byref(text_qkv), ctypes.byref(video_out),
                                ctypes.byref(text_out), compute, _s(stream)), "awa_forward")

    def forward_noalloc(self, video_qkv: AwaBlob, text_qkv: AwaBlob, video_out: AwaBlob, text_out: AwaBlob,
                        compute: int, stream: Optional[Stream] = None) -> int:
        """awa_forward_noalloc; returns its code (callers check rejections)."""
        return lib().awa_forward_noalloc(self.h, ctypes.byref(video_qkv), ctypes.byref(text_qkv),
                                         ctypes.byref(video_out), ctypes.byref(text_out), compute, _s(stream))

    def forward_qknorm(self, video_qkv: AwaBlob, text_qkv: AwaBlob, norm: AwaQkNorm, video_out: AwaBlob,
                       text_out: AwaBlob, compute: int = COMPUTE_F32, stream: Optional[Stream] = None) -> None:
        check(lib().awa_forward_qknorm(self.h, ctypes.byref(video_qkv), ctypes.byref(text_qkv), ctypes.byref(norm),
                                       ctypes.byref(video_out), ctypes.byref(text_out), compute, _s(stream)),
              "awa_forward_qknorm")

    def pack(self, video_qkv: AwaBlob, text_qkv: AwaBlob, packed: AwaBlob, cu: AwaBlob,
             stream: Optional[Stream] = None) -> None:
        check(lib().awa_pack(self.h, ctypes.byref(video_qkv), ctypes.byref(text_qkv), ctypes.byref(packed),
                             ctypes.byref(cu), _s(stream)), "awa_pack")

    def mmrope(self, inp: AwaBlob, out: AwaBlob, stream: Optional[Stream] = None) -> None:
        check(lib().awa_mmrope(self.h, ctypes.byref(inp), ctypes.byref(out), _s(stream)), "awa_mmrope")

    def window_attention(self, inp: AwaBlob, out: AwaBlob, compute: int, stream: Optional[Stream] = None) -> None:
        check(lib().awa_window_attention(self.h, ctypes.byref(inp), ctypes.byref(out), compute, _s(stream)),
              "awa_window_attention")

    def unpack(self, packed: AwaBlob, video_out: AwaBlob, text_out: AwaBlob, stream: Optional[Stream] = None) -> None:
        check(lib().awa_unpack(self.h, ctypes.byref(packed), ctypes.byref(video_out), ctypes.byref(text_out),
                               _s(stream)), "awa_unpack")


class DitBlock:
    """One DiT block around the AWA layer (awa_dit_block_*)."""

    def __init__(self, t: int, h: int, w: int, nt: int, nh: int, nw: int, text_tokens: int, shifted: bool,
                 heads: int, head_dim: int, hidden: int, mlp_hidden: int, last_layer: bool, precision: int,
                 norm_eps: float = 1e-5):
        self.desc = AwaDitBlockDesc(t, h, w, nt, nh, nw, text_tokens, int(shifted), heads, head_dim, hidden,
                                    mlp_hidden, int(last_layer), precision, norm_eps)
        p = ctypes.c_void_p()
        check(lib().awa_dit_block_create(ctypes.byref(self.desc), ctypes.byref(p)), "awa_dit_block_create")
        self.handle = p.value

    def forward(self, video_weights: AwaDitBranchWeights, text_weights: AwaDitBranchWeights, video: int, text: int,
                emb: int, video_out: int, text_out: int, stream: Optional["Stream"] = None) -> None:
        check(lib().awa_dit_block_forward(ctypes.c_void_p(self.handle), ctypes.byref(video_weights),
                                          ctypes.byref(text_weights), ctypes.c_void_p(video), ctypes.c_void_p(text),
                                          ctypes.c_void_p(emb), ctypes.c_void_p(video_out),
                                          ctypes.c_void_p(text_out), _s(stream)), "awa_dit_block_forward")

    def destroy(self) -> None:
        if self.handle:
            lib().awa_dit_block_destroy(ctypes.c_void_p(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class DitStack:
    """The DiT step's block loop (awa_dit_stack_*): full blocks with the fp32/bf16 dispatch."""

    def __init__(self, t: int, h: int, w: int, nt: int, nh: int, nw: int, text_tokens: int, blocks: int,
                 fp32_prefix_blocks: int, heads: int, head_dim: int, hidden: int, mlp_hidden: int,
                 norm_eps: float = 1e-5):
        self.desc = AwaDitStackDesc(t, h, w, nt, nh, nw, text_tokens, blocks, fp32_prefix_blocks, heads, head_dim,
                                    hidden, mlp_hidden, norm_eps)
        p = ctypes.c_void_p()
        check(lib().awa_dit_stack_create(ctypes.byref(self.desc), ctypes.byref(p)), "awa_dit_stack_create")
        self.handle = p.value
        self.blocks = blocks

    def run(self, video_weights: Sequence[AwaDitBranchWeights], text_weights: Sequence[AwaDitBranchWeights],
            video: int, text: int, emb: int, video_out: int, text_out: int,
            stream: Optional["Stream"] = None) -> None:
        arr = AwaDitBranchWeights * self.blocks
        check(lib().awa_dit_stack_run(ctypes.c_void_p(self.handle), arr(*video_weights), arr(*text_weights),
                                      ctypes.c_void_p(video), ctypes.c_void_p(text), ctypes.c_void_p(emb),
                                      ctypes.c_void_p(video_out), ctypes.c_void_p(text_out), _s(stream)),
              "awa_dit_stack_run")

    def set_profiling(self, enabled: bool) -> None:
        check(lib().awa_dit_stack_set_profiling(ctypes.c_void_p(self.handle), int(enabled)),
              "awa_dit_stack_set_profiling")

    def block_times(self) -> np.ndarray:
        t = (ctypes.c_float * self.blocks)()
        check(lib().awa_dit_stack_block_times(ctypes.c_void_p(self.handle), t), "awa_dit_stack_block_times")
        return np.array(t[:], np.float64)

    def destroy(self) -> None:
        if self.handle:
            lib().awa_dit_stack_destroy(ctypes.c_void_p(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class AttentionStack:
    """The DiT attention stack (awa_stack_*): per-block AWA with the fp32/bf16 dispatch."""

    def __init__(self, t: int, h: int, w: int, nt: int, nh: int, nw: int, text_tokens: int, blocks: int = 32,
                 fp32_prefix_blocks: int = 9, heads: int = 20, head_dim: int = 128):
        self.desc = AwaStackDesc(t, h, w, nt, nh, nw, text_tokens, blocks, fp32_prefix_blocks, heads, head_dim)
        p = ctypes.c_void_p()
        check(lib().awa_stack_create(ctypes.byref(self.desc), ctypes.byref(p)), "awa_stack_create")
        self.handle = p.value
        self.blocks = blocks

    def run(self, video_qkv: Sequence[int], text_qkv: Sequence[int], video_out: Sequence[int],
            text_out: Sequence[int], stream: Optional[Stream] = None) -> None:
        arr = ctypes.c_void_p * self.blocks
        check(lib().awa_stack_run(ctypes.c_void_p(self.handle), arr(*video_qkv), arr(*text_qkv), arr(*video_out),
                                  arr(*text_out), _s(stream)), "awa_stack_run")

    def set_profiling(self, enabled: bool) -> None:
        check(lib().awa_stack_set_profiling(ctypes.c_void_p(self.handle), int(enabled)), "awa_stack_set_profiling")

    def set_graph(self, enabled: bool) -> None:
        """Replay steps through a captured HIP graph (default on)."""
        check(lib().awa_stack_set_graph(ctypes.c_void_p(self.handle), int(enabled)), "awa_stack_set_graph")

    def block_times(self):
        att = (ctypes.c_float * self.blocks)()
        blk = (ctypes.c_float * self.blocks)()
        check(lib().awa_stack_block_times(ctypes.c_void_p(self.handle), att, blk), "awa_stack_block_times")
        return np.array(att[:], np.float64), np.array(blk[:], np.float64)

    def block_flops(self) -> np.ndarray:
        f = (ctypes.c_double * self.blocks)()
        check(lib().awa_stack_block_flops(ctypes.c_void_p(self.handle), f), "awa_stack_block_flops")
        return np.array(f[:], np.float64)

    def destroy(self) -> None:
        if self.handle:
            lib().awa_stack_destroy(ctypes.c_void_p(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


def rmsnorm(inp: AwaBlob, gamma_ptr: Optional[int], eps: float, out: AwaBlob, stream: Optional[Stream] = None) -> None:
    check(lib().awa_rmsnorm(ctypes.byref(inp), gamma_ptr, eps, ctypes.byref(out), _s(stream)), "awa_rmsnorm")


def qkv_concat(q: AwaBlob, k: AwaBlob, v: AwaBlob, out: AwaBlob, stream: Optional[Stream] = None) -> None:
    """DitQKVConcat: fp32 q, k and fp32/bf16 v, each Mat(d, H, N), into fp32 Mat(d, 3H, N)."""
    check(lib().awa_qkv_concat(ctypes.byref(q), ctypes.byref(k), ctypes.byref(v), ctypes.byref(out), _s(stream)),
          "awa_qkv_concat")


def cast(inp: AwaBlob, out: AwaBlob, stream: Optional[Stream] = None) -> None:
    check(lib().awa_cast(ctypes.byref(inp), ctypes.byref(out), _s(stream)), "awa_cast")


# ---- numpy helpers for bf16 bit patterns ----

def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round to nearest even, as the device does."""
    b = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) & 0xFFFF
    return r.astype(np.uint16)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)
