"""ctypes/numpy view of the CPU oracle (test infrastructure only).

Only tests, the smoke check and the CPU-baseline leg of ``bench.py`` use this
module, always as the checker. It wraps ``liboracle_awa.so`` built from
``awa_oracle.cpp`` (``make -C oracle``); every function there cites the
reference code it restates.
"""

from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_REF = None

_i = ctypes.c_int
_ll = ctypes.c_longlong
_p = ctypes.c_void_p


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        path = os.path.join(HERE, "liboracle_awa.so")
        if not os.path.exists(path):
            raise RuntimeError(f"oracle library missing: {path} (run `make -C oracle`)")
        _LIB = ctypes.CDLL(path)
        _LIB.orc_set_num_threads.argtypes = [_i]
        _LIB.orc_python_round_positive.argtypes = [ctypes.c_double]
        _LIB.orc_make_windows.argtypes = [_i] * 7 + [_p, _i]
        _LIB.orc_map_sizes.argtypes = [_i] * 8 + [_p]
        _LIB.orc_build_maps.argtypes = [_i] * 8 + [_p] * 5
        _LIB.orc_rope_table.argtypes = [_i] * 9 + [_p]
        _LIB.orc_pack_forward.argtypes = [_p, _ll, _ll, _p, _ll, _ll, _p, _i, _p, _i, _i, _i, _i, _p, _p]
        _LIB.orc_mmrope_forward.argtypes = [_p, _p, _i, _i, _i, _i, _p]
        _LIB.orc_attention_cpu.argtypes = [_p, _p, _i, _i, _i, _p]
        _LIB.orc_attention_kahan.argtypes = [_p, _p, _i, _i, _i, _p]
        _LIB.orc_unpack_forward.argtypes = [_p, _p, _i, _p, _i, _i, _i, _i, _i, _p, _p]
        _LIB.orc_fill_gaussian.argtypes = [_p, _ll, ctypes.c_uint, ctypes.c_ulonglong]
        _LIB.orc_seed_seq_words.argtypes = [ctypes.c_uint, ctypes.c_ulonglong, _p]
        _LIB.orc_round_bf16.argtypes = [_p, _p, _ll]
        _LIB.orc_awa_layer.argtypes = [_p, _p] + [_i] * 13 + [_p, _p]
        _LIB.orc_rmsnorm.argtypes = [_p, _ll, _i, _p, ctypes.c_float, _p]
    return _LIB


def ref_sampler():
    """The reference's own fill_gaussian_noise built in oracle/_ref, or None."""
    global _REF
    if _REF is None:
        path = os.path.join(HERE, "_ref", "libref_sampler.so")
        if not os.path.exists(path):
            return None
        _REF = ctypes.CDLL(path)
        _REF.ref_fill_gaussian_noise.argtypes = [_p, ctypes.c_ulonglong, ctypes.c_uint, ctypes.c_ulonglong]
    return _REF


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


@dataclass(frozen=True)
class Geometry:
    """One AWA layer's parameters (the reference's layer params 0-7)."""

    t: int
    h: int
    w: int
    nt: int
    nh: int
    nw: int
    text_tokens: int
    shifted: bool

    @property
    def args(self):
        return (self.t, self.h, self.w, self.nt, self.nh, self.nw)

    @property
    def source_tokens(self) -> int:
        return self.t * self.h * self.w


def set_num_threads(threads: int) -> None:
    """Threads of the oracle's (window, head) loops; 1 = the reference's single thread."""
    if lib().orc_set_num_threads(int(threads)) != 0:
        raise ValueError("threads must be >= 1")


def python_round_positive(x: float) -> int:
    return lib().orc_python_round_positive(float(x))


def make_windows(g: Geometry) -> np.ndarray:
    cap = 1 << 16
    out = np.zeros((cap, 6), dtype=np.int32)
    n = lib().orc_make_windows(*g.args, int(g.shifted), _ptr(out), cap)
    if n < 0:
        raise ValueError("invalid window arguments")
    return out[:n].copy()


@dataclass
class Maps:
    sequence_index: np.ndarray
    cu_seqlens: np.ndarray
    video_positions: np.ndarray
    text_positions: np.ndarray
    target: np.ndarray
    status: int

    @property
    def window_count(self) -> int:
        return len(self.cu_seqlens) - 1

    @property
    def sequence_tokens(self) -> int:
        return len(self.sequence_index)


def build_maps(g: Geometry) -> Maps:
    sizes = np.zeros(2, dtype=np.int32)
    lib().orc_map_sizes(*g.args, g.text_tokens, int(g.shifted), _ptr(sizes))
    S, nwin = int(sizes[0]), int(sizes[1])
    N = g.source_tokens
    seq = np.zeros(S, np.int32)
    cu = np.zeros(nwin + 1, np.int32)
    vpos = np.zeros(N, np.int32)
    tpos = np.zeros(nwin * g.text_tokens, np.int32)
    target = np.zeros(N, np.int32)
    st = lib().orc_build_maps(*g.args, g.text_tokens, int(g.shifted), _ptr(seq), _ptr(cu), _ptr(vpos),
                              _ptr(tpos), _ptr(target))
    return Maps(seq, cu, vpos, tpos, target, st)


def rope_table(g: Geometry, rope_dim: int = 126) -> np.ndarray:
    m = build_maps(g)
    out = np.zeros((m.sequence_tokens, 2 * rope_dim), np.float32)
    n = lib().orc_rope_table(*g.args, g.text_tokens, int(g.shifted), rope_dim, _ptr(out))
    if n != m.sequence_tokens:
        raise ValueError("invalid rope_dim")
    return out


def pack_forward(g: Geometry, video: np.ndarray, text: np.ndarray, heads: int, head_dim: int):
    """video [N][3][H][d], text [T_x][3][H][d] fp32 -> packed [S][3][H][d], cu float."""
    m = build_maps(g)
    video = np.ascontiguousarray(video, np.float32)
    text = np.ascontiguousarray(text, np.float32)
    row = 3 * heads * head_dim
    packed = np.zeros((m.sequence_tokens, 3, heads, head_dim), np.float32)
    cu = np.zeros(m.window_count + 1, np.float32)
    lib().orc_pack_forward(_ptr(video), row, heads * head_dim, _ptr(text), row, heads * head_dim,
                           _ptr(m.sequence_index), m.sequence_tokens, _ptr(m.cu_seqlens), m.window_count,
                           g.source_tokens, heads, head_dim, _ptr(packed), _ptr(cu))
    return packed, cu


def mmrope_forward(packed: np.ndarray, table: np.ndarray, heads: int, head_dim: int, rope_dim: int = 126):
    packed = np.ascontiguousarray(packed, np.float32)
    out = np.zeros_like(packed)
    lib().orc_mmrope_forward(_ptr(packed), _ptr(np.ascontiguousarray(table, np.float32)), packed.shape[0], heads,
                             head_dim, rope_dim, _ptr(out))
    return out


def attention(packed: np.ndarray, cu_seqlens: np.ndarray, heads: int, head_dim: int, order: str = "kahan"):
    """packed [S][3][H][d] -> [S][H][d]; order 'cpu' (loop order) or 'kahan' (shader order)."""
    packed = np.ascontiguousarray(packed, np.float32)
    cu = np.ascontiguousarray(cu_seqlens, np.int32)
    out = np.zeros((packed.shape[0], heads, head_dim), np.float32)
    fn = lib().orc_attention_cpu if order == "cpu" else lib().orc_attention_kahan
    fn(_ptr(packed), _ptr(cu), len(cu) - 1, heads, head_dim, _ptr(out))
    return out


def unpack_forward(g: Geometry, packed_out: np.ndarray, heads: int, head_dim: int, text_order: str = "gpu"):
    """packed [S][H][d] -> video [N][H][d], text [T_x][H][d]; text_order 'cpu' or 'gpu'."""
    m = build_maps(g)
    packed_out = np.ascontiguousarray(packed_out, np.float32)
    video = np.zeros((g.source_tokens, heads, head_dim), np.float32)
    text = np.zeros((g.text_tokens, heads, head_dim), np.float32)
    lib().orc_unpack_forward(_ptr(packed_out), _ptr(m.video_positions), g.source_tokens, _ptr(m.text_positions),
                             g.text_tokens, m.window_count, heads, head_dim, 0 if text_order == "cpu" else 1,
                             _ptr(video), _ptr(text))
    return video, text


def awa_layer(g: Geometry, video_qkv: np.ndarray, text_qkv: np.ndarray, heads: int, head_dim: int,
              rope_dim: int = 126, attention_order: str = "kahan", text_order: str = "gpu"):
    """Whole chain Pack -> MMRoPE -> WindowAttention -> Unpack on fp32 inputs."""
    video_qkv = np.ascontiguousarray(video_qkv, np.float32)
    text_qkv = np.ascontiguousarray(text_qkv, np.float32)
    video = np.zeros((g.source_tokens, heads, head_dim), np.float32)
    text = np.zeros((g.text_tokens, heads, head_dim), np.float32)
    rc = lib().orc_awa_layer(_ptr(video_qkv), _ptr(text_qkv), *g.args, g.text_tokens, int(g.shifted), rope_dim,
                             heads, head_dim, 0 if attention_order == "cpu" else 1,
                             0 if text_order == "cpu" else 1, _ptr(video), _ptr(text))
    if rc != 0:
        raise ValueError("oracle layer failed")
    return video, text


def rmsnorm(x: np.ndarray, gamma, eps: float) -> np.ndarray:
    """DitRMSNorm over the last axis (shader order); gamma None = no affine."""
    x = np.ascontiguousarray(x, np.float32)
    width = x.shape[-1]
    out = np.zeros_like(x)
    g = None if gamma is None else np.ascontiguousarray(gamma, np.float32)
    if g is not None and g.shape != (width,):
        raise ValueError("gamma must have the row width")
    rc = lib().orc_rmsnorm(_ptr(x), x.size // width, width, None if g is None else _ptr(g), eps, _ptr(out))
    if rc != 0:
        raise ValueError("invalid rmsnorm arguments")
    return out


def qkv_concat(q: np.ndarray, k: np.ndarray, v: np.ndarray) -> np.ndarray:
    """DitQKVConcat (src/dit/shader/dit_qkv_concat.comp:17-31): q, k, v of
    shape [tokens][heads][d] into [tokens][3 heads][d] fp32; output row y
    reads head y % heads of q (y < heads), k (y < 2 heads) or v, whose values
    are promoted exactly."""
    q, k, v = (np.asarray(a, np.float32) for a in (q, k, v))
    if q.ndim != 3 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError("q, k and v must be [tokens][heads][d] of one shape")
    tokens, heads, d = q.shape
    out = np.empty((tokens, 3 * heads, d), np.float32)
    for y in range(3 * heads):
        src = q if y < heads else (k if y < 2 * heads else v)
        out[:, y, :] = src[:, y % heads, :]
    return out


def qk_norm_inputs(video: np.ndarray, text: np.ndarray, gammas, eps: float):
    """The DiT block's q/k RMSNorm on raw QKV: video [N][3][H][d], text
    [T_x][3][H][d]; gammas (q_video, k_video, q_text, k_text) of head_dim each.
    V passes through (tools/reference/dit_block.py:280-290)."""
    q_video, k_video, q_text, k_text = gammas
    v = np.array(video, np.float32, copy=True)
    t = np.array(text, np.float32, copy=True)
    v[:, 0] = rmsnorm(v[:, 0], q_video, eps)
    v[:, 1] = rmsnorm(v[:, 1], k_video, eps)
    t[:, 0] = rmsnorm(t[:, 0], q_text, eps)
    t[:, 1] = rmsnorm(t[:, 1], k_text, eps)
    return v, t


def fill_gaussian(count: int, seed: int, stream: int = 0) -> np.ndarray:
    out = np.zeros(count, np.float32)
    if lib().orc_fill_gaussian(_ptr(out), count, seed, stream) != 0:
        raise ValueError("invalid noise request")
    return out


def seed_seq_words(seed: int, stream: int) -> np.ndarray:
    out = np.zeros(624, np.uint32)
    lib().orc_seed_seq_words(seed, stream, _ptr(out))
    return out


def round_bf16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(x.shape, np.uint16)
    lib().orc_round_bf16(_ptr(x), _ptr(out), x.size)
    return out


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """fp32 values rounded to the nearest bf16 (ties to even), returned as fp32."""
    return bf16_bits_to_f32(round_bf16_bits(x))


# ---- DiT block around the AWA layer (tools/reference/dit_block.py:166-207, :344-378) ----

@dataclass
class DitBranchWeights:
    """One branch's weights as fp32 host arrays: GEMM weights row-major
    [out][in] (torch Linear), proj_out_bias [hidden], norm_q / norm_k
    [head_dim], ada [6][hidden] (attn shift, scale, gate, mlp shift, scale,
    gate: AdaSingle's learned vectors, dit_block.py:166-172)."""
    qkv: np.ndarray
    proj_out: np.ndarray
    proj_out_bias: np.ndarray
    mlp_gate: np.ndarray
    mlp_in: np.ndarray
    mlp_out: np.ndarray
    norm_q: np.ndarray
    norm_k: np.ndarray
    ada: np.ndarray


def ada_vectors(emb: np.ndarray, ada: np.ndarray, layer: int):
    """(shift, scale, gate) of layer 0 (attn) or 1 (mlp): the block embedding
    read as [hidden][2][3] plus the branch's learned vectors
    (FixedAdaBranch.forward, dit_block.py:174-181)."""
    e = np.asarray(emb, np.float64).reshape(-1, 2, 3)[:, layer, :]
    a = np.asarray(ada, np.float64)
    return e[:, 0] + a[3 * layer], e[:, 1] + a[3 * layer + 1], e[:, 2] + a[3 * layer + 2]


def _rms(x: np.ndarray, eps: float) -> np.ndarray:
    """nn.RMSNorm without affine over the last axis: x / sqrt(mean(x^2) + eps)."""
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)


def dit_block(g: Geometry, video: np.ndarray, text: np.ndarray, emb: np.ndarray, wv: DitBranchWeights,
              wt: DitBranchWeights, heads: int, head_dim: int, eps: float, last_layer: bool, bf16: bool = False):
    """FixedDitBlock.forward (dit_block.py:344-378) for one block: video
    [N][hidden], text [T_x][hidden], emb [hidden*6]. Arithmetic is float64
    except the AWA layer, which is the fp32 oracle above (q/k RMSNorm, then
    Pack -> MMRoPE -> WindowAttention -> Unpack). With bf16=True the values are
    rounded to bf16 where the bf16 DiT block stores them: the inputs, the
    GEMM weights, and the output of every fused step (norm + Ada in, each
    GEMM before its bias, the AWA layer, gate + residual, SwiGLU)."""
    r = (lambda x: round_bf16(np.asarray(x, np.float32)).astype(np.float64)) if bf16 else \
        (lambda x: np.asarray(x, np.float64))
    wts = (wv, wt)
    xs = (r(video), r(text))
    modulate = (True, not last_layer)
    hd = heads * head_dim

    def lin(x, w):
        return r(x @ r(w).T)

    qkv = []
    for br in range(2):
        xa = _rms(xs[br], eps)
        if modulate[br]:
            shift, scale, _ = ada_vectors(r(emb), wts[br].ada, 0)
            xa = xa * scale + shift
        qkv.append(lin(r(xa), wts[br].qkv).reshape(-1, 3, heads, head_dim))
    gammas = (wv.norm_q, wv.norm_k, wt.norm_q, wt.norm_k)
    qv, qt = qk_norm_inputs(qkv[0].astype(np.float32), qkv[1].astype(np.float32), gammas, eps)
    av, at = awa_layer(g, qv, qt, heads, head_dim)
    att = (r(av.reshape(-1, hd)), r(at.reshape(-1, hd)))
    outs = []
    for br in range(2):
        w = wts[br]
        h = lin(att[br], w.proj_out) + np.asarray(w.proj_out_bias, np.float64)
        if not modulate[br]:
            y = r(h + xs[br])
            outs.append(r(y + y))  # the last block's text: txt_attn + txt_attn
            continue
        _, _, gate = ada_vectors(r(emb), w.ada, 0)
        y = r(h * gate + xs[br])
        shift, scale, gate = ada_vectors(r(emb), w.ada, 1)
        xm = r(_rms(y, eps) * scale + shift)
        a = lin(xm, w.mlp_gate)
        b = lin(xm, w.mlp_in)
        hidden = r(a / (1.0 + np.exp(-a)) * b)
        outs.append(r(lin(hidden, w.mlp_out) * gate + y))
    return outs[0], outs[1]
