"""Generic forward attention on the gfx950 core.

``attention(q, k, v, **mask_and_score_params) -> o`` is the one entry point
all ten variant modules call.  It validates on the host, allocates ``o`` with
torch on q's device (the reference's ownership rule, e.g.
kernels_gemini31propre_0018/bias_sliding_window_BEST.py:89), and launches
``chia_attn_fwd`` on torch's current HIP stream, asynchronously, exactly like
the reference's ``launch_kernel`` (which launches on the current stream and
leaves synchronisation to the caller, extra_bench.py:12,19).
"""
from __future__ import annotations

import ctypes
import math
import threading
import weakref
from collections import OrderedDict
from typing import Optional, Sequence, Union

import torch

from . import _lib

PerHead = Union[None, torch.Tensor, Sequence[float]]

SUPPORTED_HEAD_DIMS = (64, 128)
_VEC_CACHE_MAX = 64
_vec_cache: "OrderedDict[tuple, torch.Tensor]" = OrderedDict()
_ARGS_CACHE_MAX = 256

# The current stream's raw handle for a device index, without building a Stream
# object (the cached launch paths' largest fixed cost after the launch itself).
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _current_stream(t: torch.Tensor) -> int:
    if _raw_stream is not None:
        return _raw_stream(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream
_tls = threading.local()


def _args_cache() -> "OrderedDict[tuple, tuple]":
    cache = getattr(_tls, "args", None)
    if cache is None:
        cache = _tls.args = OrderedDict()
    return cache


def _head_key(vals: PerHead):
    """Cache key of a per-head parameter: device tensors by identity of storage
    (their values are read by the kernel at every call), host values by content."""
    if vals is None:
        return None
    if isinstance(vals, torch.Tensor):
        if vals.device.type == "cuda":
            if vals.dtype != torch.float32 or not vals.is_contiguous():
                raise TypeError("converted device vectors are not cached")  # caller takes the full path
            return ("dev", vals.data_ptr(), tuple(vals.shape))
        return ("host", tuple(vals.detach().reshape(-1).tolist()))
    if type(vals) is tuple:  # e.g. the variants' cached presets: hashed as they are
        return ("host", vals)
    return ("host", tuple(float(x) for x in vals))


def _per_head_vector(vals: PerHead, heads: int, device: torch.device, name: str,
                     positive: bool, cache: bool = True) -> Optional[torch.Tensor]:
    """float32 [heads] device vector for a per-head parameter (cached for host values
    unless `cache` is False, as while tracing with fake tensors)."""
    if vals is None:
        return None
    if isinstance(vals, torch.Tensor) and vals.device.type == "cuda":
        t = vals
        if t.shape != (heads,):
            raise ValueError(f"{name} must have shape ({heads},), got {tuple(t.shape)}")
        if t.device != device:
            raise ValueError(f"{name} is on {t.device}, tensors are on {device}")
        return t.to(torch.float32).contiguous()
    # host values: checked in Python (no tensor op, so fake-tensor tracing can run this)
    if isinstance(vals, torch.Tensor):
        if not cache:  # tracing: the values are not read on the host (nor checked)
            t = vals.detach().to(torch.float32).reshape(-1)
            if t.numel() != heads:
                raise ValueError(f"{name} must have {heads} values, got {t.numel()}")
            return t.to(device)
        vals = vals.detach().reshape(-1).tolist()
    host = [float(x) for x in vals]
    if len(host) != heads:
        raise ValueError(f"{name} must have {heads} values, got {len(host)}")
    if not all(math.isfinite(x) for x in host):
        raise ValueError(f"{name} must be finite")
    if positive and not all(x > 0 for x in host):
        raise ValueError(f"{name} must be > 0")
    if not cache:
        return torch.tensor(host, dtype=torch.float32).to(device)  # a host constant, then a copy (traceable)
    key = (name, device.index, tuple(host))
    cached = _vec_cache.get(key)
    if cached is None:
        cached = torch.tensor(host, dtype=torch.float32).to(device)
        _vec_cache[key] = cached
        if len(_vec_cache) > _VEC_CACHE_MAX:
            _vec_cache.popitem(last=False)
    else:
        _vec_cache.move_to_end(key)
    return cached


def _layout_ok(t: torch.Tensor) -> bool:
    if t.stride(-1) != 1:
        return False
    if any(s % 8 for s in t.stride()[:3]):
        return False
    return t.data_ptr() % 16 == 0


def make_args(*, batch: int, heads: int, seqlen: int, head_dim: int, norm: str = "softmax",
              causal: bool = True, window: int = 0, dilation: int = 1, block: int = 0, prefix: int = 0,
              scale: Optional[float] = None, softcap: float = 0.0, bias: float = 0.0,
              post_scale: float = 1.0, alibi: bool = False, head_scale: bool = False) -> _lib.AttnArgs:
    """Argument struct without tensors (for the host-only planning calls)."""
    if norm not in _lib.NORMS:
        raise ValueError(f"norm must be one of {sorted(_lib.NORMS)}, got {norm!r}")
    a = _lib.AttnArgs()
    a.norm = _lib.NORMS[norm]
    a.batch, a.heads, a.seqlen, a.head_dim = batch, heads, seqlen, head_dim
    a.causal = 1 if causal else 0
    a.window = int(window or 0)
    a.dilation = int(dilation or 1)
    a.block = int(block or 0)
    a.prefix = int(prefix or 0)
    a.scale = float(1.0 / math.sqrt(head_dim) if scale is None else scale)
    a.softcap = float(softcap or 0.0)
    a.bias = float(bias)
    a.post_scale = float(post_scale)
    # planning ignores the per-head pointers' contents; non-null marks the feature
    a.alibi_slopes = 16 if alibi else None
    a.head_scale = 16 if head_scale else None
    return a


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, norm: str = "softmax",
              causal: bool = True, window: int = 0, dilation: int = 1, block: int = 0, prefix: int = 0,
              scale: Optional[float] = None, head_scale: PerHead = None, alibi_slopes: PerHead = None,
              softcap: float = 0.0, bias: float = 0.0, post_scale: float = 1.0,
              out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Forward attention o = norm(mod(q k^T) | mask) @ v for bf16 [B, H, S, D] tensors.

    k and v may have fewer heads than q ([B, H_kv, S, D], H_kv dividing H): query head h
    then reads K/V head h // (H // H_kv) (grouped-query / multi-query attention).

    Mask: query i sees key j iff (j < prefix) or (band and block and dilation), with
    band = 0 <= i-j (< window) when causal, |i-j| < window otherwise (window=0: no limit),
    block: i//block == j//block, dilation: (i-j) % dilation == 0.
    Score: (q.k) * scale * head_scale[h] + alibi_slopes[h] * (j - i), then
    softcap * tanh(s / softcap) when softcap > 0.
    norm: "softmax" | "sigmoid" (sigmoid(s + bias) * post_scale) | "relu" (relu(s) * post_scale).
    """
    params = dict(norm=norm, causal=causal, window=window, dilation=dilation, block=block, prefix=prefix,
                  scale=scale, head_scale=head_scale, alibi_slopes=alibi_slopes, softcap=softcap, bias=bias,
                  post_scale=post_scale)
    needs_grad = torch.is_grad_enabled() and any(isinstance(t, torch.Tensor) and t.requires_grad for t in (q, k, v))
    if needs_grad or torch.compiler.is_compiling():
        # the registered operator: autograd (chia_attn::bwd) and torch.compile see one node
        if out is not None:
            raise ValueError("out= is not supported when q, k or v requires grad or under torch.compile")
        return _op_forward(q, k, v, params)[0]
    # Fast path: a call with the same shapes, layouts and parameters as an
    # earlier one reuses its validated argument struct and per-head vectors;
    # only the data pointers (and their alignment) are new.
    try:
        key = (q.shape, q.dtype, k.dtype, v.dtype, q.device, q.stride(), k.shape, k.stride(), v.shape, v.stride(),
               k.device, v.device, None if out is None else (out.shape, out.dtype, out.device, out.stride()),
               norm, causal, window, dilation, block, prefix, scale, softcap, bias, post_scale,
               _head_key(head_scale), _head_key(alibi_slopes))
    except (AttributeError, TypeError):
        key = None
    cache = _args_cache()
    entry = cache.get(key) if key is not None else None
    if entry is not None:
        a, hs, sl = entry
        o = torch.empty_like(q) if out is None else out
        ptrs = (q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr())
        if not (ptrs[0] | ptrs[1] | ptrs[2] | ptrs[3]) & 15:
            a.q, a.k, a.v, a.o = ptrs
            # device fp32 vectors are passed as they are (their values may change
            # between calls); host values were copied to the device once
            if hs is not None:
                a.head_scale = (head_scale if isinstance(head_scale, torch.Tensor) and head_scale.is_cuda
                                else hs).data_ptr()
            if sl is not None:
                a.alibi_slopes = (alibi_slopes if isinstance(alibi_slopes, torch.Tensor) and alibi_slopes.is_cuda
                                  else sl).data_ptr()
            _lib.fwd(a, _current_stream(q))
            return o

    a, hs, sl, (q_, k_, v_), o = _prepare(q, k, v, out, **params)
    with torch.cuda.device(q.device):
        stream = torch.cuda.current_stream(q.device).cuda_stream
        _lib.fwd(a, stream)
    # Cache the validated call when the tensors needed no layout change and a
    # fresh output would get the same strides as this one.
    if key is not None and q_ is q and k_ is k and v_ is v and (out is not None or o.stride() == q.stride()):
        cache[key] = (a, hs, sl)
        if len(cache) > _ARGS_CACHE_MAX:
            cache.popitem(last=False)
    return o


def _check_params(D, norm, window, dilation, block, prefix, scale, softcap) -> float:
    """Host checks of the head dim and scalar parameters; returns the resolved scale."""
    if D not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"head_dim must be one of {SUPPORTED_HEAD_DIMS}, got {D}")
    if norm not in _lib.NORMS:
        raise ValueError(f"norm must be one of {sorted(_lib.NORMS)}, got {norm!r}")
    if window < 0 or block < 0 or prefix < 0 or dilation < 1:
        raise ValueError("window, block, prefix must be >= 0 and dilation >= 1")
    if dilation > 1 and prefix > 0:
        raise ValueError("prefix cannot be combined with dilation > 1")
    sc = 1.0 / math.sqrt(D) if scale is None else float(scale)
    if not (sc > 0 and math.isfinite(sc)):
        raise ValueError(f"scale must be finite and > 0, got {scale}")
    if softcap < 0 or not math.isfinite(softcap):
        raise ValueError(f"softcap must be finite and >= 0, got {softcap}")
    return sc


def _prepare(q, k, v, out, *, norm, causal, window, dilation, block, prefix, scale, head_scale, alibi_slopes,
             softcap, bias, post_scale):
    """Validate, make the layouts the kernel takes, allocate o and fill the argument struct."""
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    if q.dim() != 4:
        raise ValueError(f"q must be 4-D [B, H, S, D], got shape {tuple(q.shape)}")
    if (k.dim() != 4 or k.shape != v.shape or k.shape[0] != q.shape[0] or k.shape[2:] != q.shape[2:]
            or k.shape[1] < 1 or q.shape[1] % k.shape[1] != 0):
        raise ValueError(f"k and v must be [B, H_kv, S, D] with H_kv dividing q's H (GQA / MQA), got "
                         f"{tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise TypeError(f"q, k, v must be bfloat16, got {q.dtype}, {k.dtype}, {v.dtype}")
    if q.device.type != "cuda" or k.device != q.device or v.device != q.device:
        raise ValueError(f"q, k, v must be on the same GPU device, got {q.device}, {k.device}, {v.device}")
    B, H, S, D = q.shape
    if min(B, H, S) < 1:
        raise ValueError(f"empty tensor shape {tuple(q.shape)}")
    sc = _check_params(D, norm, window, dilation, block, prefix, scale, softcap)

    q_, k_, v_ = (t if _layout_ok(t) else t.contiguous() for t in (q, k, v))
    if out is None:
        o = torch.empty_like(q_)
    else:
        if out.shape != q.shape or out.dtype != torch.bfloat16 or out.device != q.device:
            raise ValueError("out must be a bf16 tensor of q's shape on q's device")
        if not _layout_ok(out):
            raise ValueError("out must have unit last stride, 16-byte alignment and strides that are multiples of 8")
        o = out
    hs = _per_head_vector(head_scale, H, q.device, "head_scale", positive=True)
    sl = _per_head_vector(alibi_slopes, H, q.device, "alibi_slopes", positive=False)

    a = make_args(batch=B, heads=H, seqlen=S, head_dim=D, norm=norm, causal=causal, window=window,
                  dilation=dilation, block=block, prefix=prefix, scale=sc, softcap=softcap, bias=bias,
                  post_scale=post_scale)
    a.q, a.k, a.v, a.o = q_.data_ptr(), k_.data_ptr(), v_.data_ptr(), o.data_ptr()
    a.kv_heads = k_.shape[1] if k_.shape[1] != H else 0
    for name, t in (("q_stride", q_), ("k_stride", k_), ("v_stride", v_), ("o_stride", o)):
        st = getattr(a, name)
        st[0], st[1], st[2] = t.stride(0), t.stride(1), t.stride(2)
    a.head_scale = hs.data_ptr() if hs is not None else None
    a.alibi_slopes = sl.data_ptr() if sl is not None else None
    return a, hs, sl, (q_, k_, v_), o


def _strides3(t: torch.Tensor):
    return t.stride(0), t.stride(1), t.stride(2)


def _op_forward(q, k, v, params):
    """(o, lse) through torch.ops.chia_attn.fwd, per-head values as float32 device vectors."""
    from .library import call_fwd

    if not isinstance(q, torch.Tensor) or q.dim() != 4:
        raise ValueError("q must be a 4-D [B, H, S, D] tensor")
    p = dict(params)
    H = q.shape[1]
    # no cached device vectors while tracing (fake tensors, torch.compile)
    cache = (q.device.type == "cuda" and not torch.compiler.is_compiling()
             and not isinstance(q, torch._subclasses.fake_tensor.FakeTensor))
    p["head_scale"] = _per_head_vector(p["head_scale"], H, q.device, "head_scale", positive=True, cache=cache)
    p["alibi_slopes"] = _per_head_vector(p["alibi_slopes"], H, q.device, "alibi_slopes", positive=False,
                                         cache=cache)
    return call_fwd(q, k, v, p)


def run_backward(do, q, k, v, o, lse, params):
    """dq, dk, dv by chia_attn_bwd (lse: the forward's float32 [B, H, S], softmax only)."""
    # Fast path, as attention()'s: a call with the shapes, layouts and parameters
    # of an earlier one (per-head values arrive as float32 device vectors) reuses
    # its validated argument structs; only the data pointers are new.
    hs_in, sl_in = params["head_scale"], params["alibi_slopes"]
    try:
        key = ("bwd", q.shape, q.dtype, q.device, q.stride(), k.shape, k.dtype, k.stride(), v.shape, v.dtype,
               v.stride(), o.shape, o.dtype, o.stride(), do.shape, do.dtype, do.stride(), lse is None,
               params["norm"], params["causal"], params["window"], params["dilation"], params["block"],
               params["prefix"], params["scale"], params["softcap"], params["bias"], params["post_scale"],
               tuple(None if t is None else (tuple(t.shape), t.device) for t in (hs_in, sl_in)))
        # device vectors the full path would pass through unchanged (float32, contiguous)
        if not all(t is None or (isinstance(t, torch.Tensor) and t.is_cuda and t.dtype == torch.float32
                                 and t.is_contiguous()) for t in (hs_in, sl_in)):
            key = None
    except (AttributeError, TypeError):
        key = None
    cache = _args_cache()
    entry = cache.get(key) if key is not None else None
    if entry is not None:
        b, nbytes = entry
        a = b.fwd.contents
        ptrs = (q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr())
        if not (ptrs[0] | ptrs[1] | ptrs[2] | ptrs[3] | ptrs[4]) & 15:
            dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
            ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
            a.q, a.k, a.v, a.o = ptrs[:4]
            a.head_scale = hs_in.data_ptr() if hs_in is not None else None
            a.alibi_slopes = sl_in.data_ptr() if sl_in is not None else None
            b.dout, b.dq, b.dk, b.dv = ptrs[4], dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
            b.lse = lse.data_ptr() if lse is not None else None
            b.workspace = ws.data_ptr()
            _lib.bwd(b, _current_stream(q))
            del ws  # queued: any reuse of its memory is ordered after the launch
            return dq, dk, dv

    # q_, k_, v_ (layout copies where needed) and the per-head vectors hs, sl stay
    # referenced until the launch is queued: do_, dq, dk, dv and the workspace are
    # allocated below and must not take their memory.
    a, hs, sl, (q_, k_, v_), _ = _prepare(q, k, v, o, **params)
    do_ = do if (do.dtype == torch.bfloat16 and _layout_ok(do)) else do.to(torch.bfloat16).contiguous()
    if do_.shape != q.shape:
        raise ValueError(f"do must have q's shape {tuple(q.shape)}, got {tuple(do.shape)}")
    if (lse is None) != (params["norm"] != "softmax"):
        raise ValueError("lse is required for softmax and unused otherwise")
    dq, dk, dv = (torch.empty(t.shape, dtype=torch.bfloat16, device=t.device) for t in (q_, k_, v_))
    nbytes = _lib.bwd_workspace_size(a)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q_.device)
    b = _lib.BwdArgs(dout=do_.data_ptr(), dq=dq.data_ptr(), dk=dk.data_ptr(), dv=dv.data_ptr(),
                     lse=lse.data_ptr() if lse is not None else None, workspace=ws.data_ptr(),
                     workspace_bytes=nbytes)
    b.fwd = ctypes.pointer(a)
    for name, t in (("dout_stride", do_), ("dq_stride", dq), ("dk_stride", dk), ("dv_stride", dv)):
        st = getattr(b, name)
        st[0], st[1], st[2] = _strides3(t)
    with torch.cuda.device(q_.device):
        _lib.bwd(b, torch.cuda.current_stream(q_.device).cuda_stream)
    # Cache the validated call when no tensor needed a layout change and the
    # gradients would get the strides of fresh empty_like tensors.
    if (key is not None and q_ is q and k_ is k and v_ is v and do_ is do
            and (dq.stride(), dk.stride(), dv.stride()) == (torch.empty_like(q).stride(),
                                                            torch.empty_like(k).stride(),
                                                            torch.empty_like(v).stride())):
        cache[key] = (b, nbytes)
        if len(cache) > _ARGS_CACHE_MAX:
            cache.popitem(last=False)
    del q_, k_, v_, hs, sl, ws  # queued: any reuse of their memory is ordered after the launch
    return dq, dk, dv


# ---- FP8 (e4m3 / e5m2) operands ---------------------------------------------------

FP8_DTYPE = torch.float8_e4m3fn
FP8_MAX = 448.0
# storage formats of q, k, v: torch dtype -> (chia_attn_fp8_args.format, largest finite value)
FP8_FORMATS = {torch.float8_e4m3fn: (_lib.FP8_E4M3, 448.0), torch.float8_e5m2: (_lib.FP8_E5M2, 57344.0)}


def quantize_fp8(x: torch.Tensor, amax: Optional[float] = None, dtype: torch.dtype = FP8_DTYPE):
    """Per-tensor FP8 quantisation: (x8, descale) with x ~= x8.float() * descale;
    the scale maps max |x| (or `amax`) to the format's largest finite value
    (448 for e4m3, the default; 57344 for torch.float8_e5m2)."""
    if dtype not in FP8_FORMATS:
        raise TypeError(f"dtype must be torch.float8_e4m3fn or torch.float8_e5m2, got {dtype}")
    top = FP8_FORMATS[dtype][1]
    if amax is None:
        a = float(x.detach().abs().max()) if x.numel() else 0.0
    else:
        a = float(amax)
    descale = a / top if a > 0 and math.isfinite(a) else 1.0
    x8 = (x.float() / descale).clamp(-top, top).to(dtype)
    return x8, descale


def attention_fp8(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, q_descale: float = 1.0,
                  k_descale: float = 1.0, v_descale: float = 1.0, norm: str = "softmax", causal: bool = True,
                  window: int = 0, dilation: int = 1, block: int = 0, prefix: int = 0,
                  scale: Optional[float] = None, head_scale: PerHead = None, alibi_slopes: PerHead = None,
                  softcap: float = 0.0, bias: float = 0.0, post_scale: float = 1.0,
                  out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """attention() on float8 q, k, v ([B, H, S, D] / [B, H_kv, S, D]), all three
    torch.float8_e4m3fn or all three torch.float8_e5m2, with per-tensor descales
    (real = stored * descale); returns bf16 o.  Both products run on the gfx950
    FP8 matrix path (chia_attn_fwd_fp8).  The attention weights P are rounded
    to e4m3 (round to nearest even) for the P V product, per normaliser:
      softmax  2^(x - m + 4) with a running max m that moves when a tile's max
               exceeds it by more than 4, so every weight is <= 2^8; the 2^4
               factor cancels in the row sum;
      sigmoid  256 * sigmoid(s + bias), the 256 divided out of o;
      ReLU     relu(s) clamped to 448 (e4m3's largest value) and unscaled: a
               score above 448 saturates, a weight below 2^-9 (e4m3's smallest
               subnormal) becomes 0.  Plain scores (q.k / sqrt(D)) stay far
               below 448; large softcaps or non-causal ALiBi distances can
               exceed it.
    Forward only."""
    # Fast path, as in attention(): a call with the same shapes, layouts, formats
    # and parameters as an earlier one reuses its argument structs; the data
    # pointers and descales are new.
    try:
        key = ("fp8", q.shape, q.dtype, k.dtype, v.dtype, q.device, q.stride(), k.shape, k.stride(), v.shape,
               v.stride(), k.device, v.device, None if out is None else (out.shape, out.dtype, out.device, out.stride()),
               norm, causal, window, dilation, block, prefix, scale, softcap, bias, post_scale,
               _head_key(head_scale), _head_key(alibi_slopes))
    except (AttributeError, TypeError):
        key = None
    cache = _args_cache()
    entry = cache.get(key) if key is not None else None
    if entry is not None:
        descales = (float(q_descale), float(k_descale), float(v_descale))
        if all(d > 0 and math.isfinite(d) for d in descales):
            a, f, hs, sl = entry
            o = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device) if out is None else out
            ptrs = (q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr())
            if not (ptrs[0] | ptrs[1] | ptrs[2] | ptrs[3]) & 15:
                a.q, a.k, a.v, a.o = ptrs
                if hs is not None:
                    a.head_scale = (head_scale if isinstance(head_scale, torch.Tensor) and head_scale.is_cuda
                                    else hs).data_ptr()
                if sl is not None:
                    a.alibi_slopes = (alibi_slopes if isinstance(alibi_slopes, torch.Tensor) and alibi_slopes.is_cuda
                                      else sl).data_ptr()
                f.q_descale, f.k_descale, f.v_descale = descales
                _lib.fwd_fp8(f, _current_stream(q))
                return o

    _check_fp8(q, k, v, 4)
    B, H, S, D = q.shape
    if (k.shape != v.shape or k.shape[0] != B or k.shape[2:] != q.shape[2:] or k.shape[1] < 1
            or H % k.shape[1] != 0):
        raise ValueError(f"k and v must be [B, H_kv, S, D] with H_kv dividing q's H, got {tuple(q.shape)}, "
                         f"{tuple(k.shape)}, {tuple(v.shape)}")
    if q.device.type != "cuda" or k.device != q.device or v.device != q.device:
        raise ValueError("q, k, v must be on the same GPU device")
    if min(B, H, S) < 1:
        raise ValueError(f"empty tensor shape {tuple(q.shape)}")
    for name, d in (("q_descale", q_descale), ("k_descale", k_descale), ("v_descale", v_descale)):
        if not (float(d) > 0 and math.isfinite(float(d))):
            raise ValueError(f"{name} must be finite and > 0, got {d}")
    sc = _check_params(D, norm, window, dilation, block, prefix, scale, softcap)

    def fp8_layout_ok(t):
        return t.stride(-1) == 1 and all(s % 16 == 0 for s in t.stride()[:3]) and t.data_ptr() % 16 == 0

    q_, k_, v_ = (t if fp8_layout_ok(t) else t.contiguous() for t in (q, k, v))
    if out is None:
        o = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)
    else:
        if out.shape != q.shape or out.dtype != torch.bfloat16 or out.device != q.device or not _layout_ok(out):
            raise ValueError("out must be a bf16 tensor of q's shape on q's device with unit last stride")
        o = out
    hs = _per_head_vector(head_scale, H, q.device, "head_scale", positive=True)
    sl = _per_head_vector(alibi_slopes, H, q.device, "alibi_slopes", positive=False)
    a = make_args(batch=B, heads=H, seqlen=S, head_dim=D, norm=norm, causal=causal, window=window,
                  dilation=dilation, block=block, prefix=prefix, scale=sc, softcap=softcap, bias=bias,
                  post_scale=post_scale)
    a.q, a.k, a.v, a.o = q_.data_ptr(), k_.data_ptr(), v_.data_ptr(), o.data_ptr()
    a.kv_heads = k_.shape[1] if k_.shape[1] != H else 0
    for name, t in (("q_stride", q_), ("k_stride", k_), ("v_stride", v_), ("o_stride", o)):
        st = getattr(a, name)
        st[0], st[1], st[2] = t.stride(0), t.stride(1), t.stride(2)
    a.head_scale = hs.data_ptr() if hs is not None else None
    a.alibi_slopes = sl.data_ptr() if sl is not None else None
    f = _lib.Fp8Args(format=FP8_FORMATS[q.dtype][0], attn=ctypes.pointer(a), q_descale=float(q_descale),
                     k_descale=float(k_descale), v_descale=float(v_descale))
    with torch.cuda.device(q.device):
        _lib.fwd_fp8(f, torch.cuda.current_stream(q.device).cuda_stream)
    # cache the validated call when the tensors needed no layout change (o is
    # always a fresh contiguous tensor or the caller's `out`, whose strides are
    # part of the key)
    if key is not None and q_ is q and k_ is k and v_ is v:
        cache[key] = (a, f, hs, sl)
        if len(cache) > _ARGS_CACHE_MAX:
            cache.popitem(last=False)
    return o


def _check_fp8(q, k, v, dims: int):
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not isinstance(t, torch.Tensor) or t.dtype not in FP8_FORMATS:
            raise TypeError(f"{name} must be a torch.float8_e4m3fn or torch.float8_e5m2 tensor, got "
                            f"{getattr(t, 'dtype', type(t).__name__)}")
        if t.dtype != q.dtype:
            raise TypeError(f"q, k and v must share one FP8 format, got {q.dtype} and {t.dtype}")
        if t.dim() != dims:
            raise ValueError(f"{name} must be {dims}-D, got shape {tuple(t.shape)}")


def attention_fp8_varlen(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens: torch.Tensor,
                         max_seqlen: Optional[int] = None, *, q_descale: float = 1.0, k_descale: float = 1.0,
                         v_descale: float = 1.0, norm: str = "softmax", causal: bool = True, window: int = 0,
                         dilation: int = 1, block: int = 0, prefix: int = 0, scale: Optional[float] = None,
                         head_scale: PerHead = None, alibi_slopes: PerHead = None, softcap: float = 0.0,
                         bias: float = 0.0, post_scale: float = 1.0,
                         out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """attention_fp8() over a packed batch: q [T, H, D], k / v [T, H_kv, D] float8
    (one format for the three), cu_seqlens [B + 1] token offsets as for
    attention_varlen(); returns bf16 o [T, H, D].  Forward only."""
    _check_fp8(q, k, v, 3)
    T, H, D = q.shape
    if (k.shape != v.shape or k.shape[0] != T or k.shape[2] != D or k.shape[1] < 1 or H % k.shape[1] != 0):
        raise ValueError(f"k and v must be [T, H_kv, D] with H_kv dividing q's H, got {tuple(q.shape)}, "
                         f"{tuple(k.shape)}, {tuple(v.shape)}")
    if q.device.type != "cuda" or k.device != q.device or v.device != q.device:
        raise ValueError("q, k, v must be on the same GPU device")
    for name, d in (("q_descale", q_descale), ("k_descale", k_descale), ("v_descale", v_descale)):
        if not (float(d) > 0 and math.isfinite(float(d))):
            raise ValueError(f"{name} must be finite and > 0, got {d}")
    if T == 0:
        check_cu_seqlens(cu_seqlens, 0, max_seqlen)
        return torch.empty(q.shape, dtype=torch.bfloat16, device=q.device) if out is None else out
    B, S, cu, order = _cu_plan(cu_seqlens, T, max_seqlen, q.device)
    sc = _check_params(D, norm, window, dilation, block, prefix, scale, softcap)

    def layout_ok(t):
        return t.stride(-1) == 1 and t.stride(0) % 16 == 0 and t.stride(1) % 16 == 0 and t.data_ptr() % 16 == 0

    q_, k_, v_ = (t if layout_ok(t) else t.contiguous() for t in (q, k, v))
    if out is None:
        o = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)
    else:
        if out.shape != q.shape or out.dtype != torch.bfloat16 or out.device != q.device or not _layout_ok_packed(out):
            raise ValueError("out must be a bf16 [T, H, D] tensor like q with unit last stride and 16-byte alignment")
        o = out
    hs = _per_head_vector(head_scale, H, q.device, "head_scale", positive=True)
    sl = _per_head_vector(alibi_slopes, H, q.device, "alibi_slopes", positive=False)
    a = make_args(batch=B, heads=H, seqlen=max(S, 1), head_dim=D, norm=norm, causal=causal, window=window,
                  dilation=dilation, block=block, prefix=prefix, scale=sc, softcap=softcap, bias=bias,
                  post_scale=post_scale)
    a.q, a.k, a.v, a.o = q_.data_ptr(), k_.data_ptr(), v_.data_ptr(), o.data_ptr()
    a.kv_heads = k_.shape[1] if k_.shape[1] != H else 0
    for name, t in (("q_stride", q_), ("k_stride", k_), ("v_stride", v_), ("o_stride", o)):
        st = getattr(a, name)
        st[0], st[1], st[2] = 0, t.stride(1), t.stride(0)
    a.head_scale = hs.data_ptr() if hs is not None else None
    a.alibi_slopes = sl.data_ptr() if sl is not None else None
    a.cu_seqlens = cu.data_ptr()
    a.seq_order = order.data_ptr()
    f = _lib.Fp8Args(format=FP8_FORMATS[q.dtype][0], attn=ctypes.pointer(a), q_descale=float(q_descale),
                     k_descale=float(k_descale), v_descale=float(v_descale))
    with torch.cuda.device(q.device):
        _lib.fwd_fp8(f, torch.cuda.current_stream(q.device).cuda_stream)
    del hs, sl, cu, order  # the launch is queued; torch's allocator orders any reuse after it on this stream
    return o


# ---- packed variable-length batches -------------------------------------------

def _layout_ok_packed(t: torch.Tensor) -> bool:
    return t.stride(-1) == 1 and t.stride(0) % 8 == 0 and t.stride(1) % 8 == 0 and t.data_ptr() % 16 == 0


def check_cu_seqlens(cu_seqlens, total: int, max_seqlen: Optional[int] = None) -> tuple:
    """Host check of packed-sequence offsets: a 1-D integer tensor [B + 1] with
    cu[0] = 0, non-decreasing, cu[B] = total tokens.  Returns (B, max length)
    (max_seqlen if given, which must be >= every length).  Reads the values on the
    host (a device tensor is copied back: one synchronisation)."""
    if not isinstance(cu_seqlens, torch.Tensor) or cu_seqlens.dim() != 1 or cu_seqlens.numel() < 2:
        raise ValueError("cu_seqlens must be a 1-D tensor of batch + 1 token offsets")
    if cu_seqlens.dtype.is_floating_point or cu_seqlens.dtype == torch.bool:
        raise TypeError(f"cu_seqlens must be an integer tensor, got {cu_seqlens.dtype}")
    host = cu_seqlens.detach().to("cpu", torch.int64)
    lens = host[1:] - host[:-1]
    if int(host[0]) != 0 or bool((lens < 0).any()) or int(host[-1]) != total:
        raise ValueError(f"cu_seqlens must start at 0, be non-decreasing and end at the {total} packed tokens")
    if total >= (1 << 31):
        raise ValueError("at most 2^31 - 1 packed tokens")
    longest = int(lens.max())
    if max_seqlen is not None:
        if int(max_seqlen) < longest:
            raise ValueError(f"max_seqlen {max_seqlen} is shorter than the longest sequence ({longest})")
        longest = int(max_seqlen)
    return int(lens.numel()), longest


_CU_CACHE_MAX = 32
_cu_cache: "OrderedDict[tuple, tuple]" = OrderedDict()


def _cu_plan(cu_seqlens, total: int, max_seqlen: Optional[int], device):
    """(B, max length, int32 device offsets, device dispatch order) for a checked
    cu_seqlens.  The check reads the offsets on the host (a device tensor: one
    synchronisation); the result is cached per tensor storage and version, so a
    cu_seqlens reused unchanged (every layer of a model) is checked once.  The
    order puts the longest sequences first (a shorter tail of the launch)."""
    key = None
    if isinstance(cu_seqlens, torch.Tensor) and not torch.compiler.is_compiling():
        # the same live tensor object (a weak reference guards against a new
        # tensor at a recycled id) at the same version
        key = (id(cu_seqlens), cu_seqlens._version, total, max_seqlen, str(device))
        hit = _cu_cache.get(key)
        if hit is not None and hit[0]() is cu_seqlens:
            _cu_cache.move_to_end(key)
            return hit[1]
    B, S = check_cu_seqlens(cu_seqlens, total, max_seqlen)
    host = cu_seqlens.detach().to("cpu", torch.int64)
    order = torch.argsort(host[1:] - host[:-1], descending=True, stable=True).to(torch.int32).to(device)
    cu = host.to(torch.int32).to(device)
    out = (B, S, cu, order)
    if key is not None:
        _cu_cache[key] = (weakref.ref(cu_seqlens), out)
        if len(_cu_cache) > _CU_CACHE_MAX:
            _cu_cache.popitem(last=False)
    return out


def _prepare_varlen(q, k, v, cu_seqlens, max_seqlen, out, *, norm, causal, window, dilation, block, prefix, scale,
                    head_scale, alibi_slopes, softcap, bias, post_scale):
    """_prepare for packed q [T, H, D], k / v [T, H_kv, D]; also returns the int32
    device copy of cu_seqlens the argument struct points at (keep it alive)."""
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not isinstance(t, torch.Tensor) or t.dim() != 3:
            raise ValueError(f"{name} must be a packed 3-D [T, heads, D] tensor")
    T, H, D = q.shape
    if (k.shape != v.shape or k.shape[0] != T or k.shape[2] != D or k.shape[1] < 1 or H % k.shape[1] != 0):
        raise ValueError(f"k and v must be [T, H_kv, D] with H_kv dividing q's H, got {tuple(q.shape)}, "
                         f"{tuple(k.shape)}, {tuple(v.shape)}")
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise TypeError(f"q, k, v must be bfloat16, got {q.dtype}, {k.dtype}, {v.dtype}")
    if q.device.type != "cuda" or k.device != q.device or v.device != q.device:
        raise ValueError(f"q, k, v must be on the same GPU device, got {q.device}, {k.device}, {v.device}")
    B, S, cu, order = _cu_plan(cu_seqlens, T, max_seqlen, q.device)
    sc = _check_params(D, norm, window, dilation, block, prefix, scale, softcap)
    q_, k_, v_ = (t if _layout_ok_packed(t) else t.contiguous() for t in (q, k, v))
    if out is None:
        o = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)
    else:
        if out.shape != q.shape or out.dtype != torch.bfloat16 or out.device != q.device or not _layout_ok_packed(out):
            raise ValueError("out must be a bf16 [T, H, D] tensor like q with unit last stride and 16-byte alignment")
        o = out
    hs = _per_head_vector(head_scale, H, q.device, "head_scale", positive=True)
    sl = _per_head_vector(alibi_slopes, H, q.device, "alibi_slopes", positive=False)
    a = make_args(batch=B, heads=H, seqlen=max(S, 1), head_dim=D, norm=norm, causal=causal, window=window,
                  dilation=dilation, block=block, prefix=prefix, scale=sc, softcap=softcap, bias=bias,
                  post_scale=post_scale)
    a.q, a.k, a.v, a.o = q_.data_ptr(), k_.data_ptr(), v_.data_ptr(), o.data_ptr()
    a.kv_heads = k_.shape[1] if k_.shape[1] != H else 0
    for name, t in (("q_stride", q_), ("k_stride", k_), ("v_stride", v_), ("o_stride", o)):
        st = getattr(a, name)
        st[0], st[1], st[2] = 0, t.stride(1), t.stride(0)
    a.head_scale = hs.data_ptr() if hs is not None else None
    a.alibi_slopes = sl.data_ptr() if sl is not None else None
    a.cu_seqlens = cu.data_ptr()
    a.seq_order = order.data_ptr()
    return a, (hs, sl, cu, order), (q_, k_, v_), o


def attention_varlen(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens: torch.Tensor,
                     max_seqlen: Optional[int] = None, *, norm: str = "softmax", causal: bool = True,
                     window: int = 0, dilation: int = 1, block: int = 0, prefix: int = 0,
                     scale: Optional[float] = None, head_scale: PerHead = None, alibi_slopes: PerHead = None,
                     softcap: float = 0.0, bias: float = 0.0, post_scale: float = 1.0,
                     out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """attention() over a packed batch of variable-length sequences.

    q [T, H, D], k / v [T, H_kv, D] bf16 on the GPU; cu_seqlens [B + 1] integer
    token offsets (sequence b is tokens cu_seqlens[b] .. cu_seqlens[b+1]-1; empty
    sequences allowed).  Every sequence is attended on its own, with the mask and
    ALiBi positions counted from its first token; the parameters are attention()'s.
    Returns o [T, H, D].  cu_seqlens is checked on the host (a device tensor is
    copied back: one synchronisation), once per tensor and version -- reusing
    the same unchanged tensor skips it; max_seqlen defaults to the longest sequence.
    """
    params = dict(norm=norm, causal=causal, window=window, dilation=dilation, block=block, prefix=prefix,
                  scale=scale, head_scale=head_scale, alibi_slopes=alibi_slopes, softcap=softcap, bias=bias,
                  post_scale=post_scale)
    needs_grad = torch.is_grad_enabled() and any(isinstance(t, torch.Tensor) and t.requires_grad for t in (q, k, v))
    if needs_grad or torch.compiler.is_compiling():
        if out is not None:
            raise ValueError("out= is not supported when q, k or v requires grad or under torch.compile")
        return _op_forward_varlen(q, k, v, cu_seqlens, max_seqlen, params)[0]
    if isinstance(q, torch.Tensor) and q.dim() == 3 and q.shape[0] == 0:
        check_cu_seqlens(cu_seqlens, 0, max_seqlen)
        return torch.empty_like(q) if out is None else out
    a, keep, qkv, o = _prepare_varlen(q, k, v, cu_seqlens, max_seqlen, out, **params)
    with torch.cuda.device(q.device):
        _lib.fwd(a, torch.cuda.current_stream(q.device).cuda_stream)
    del keep, qkv  # the launch is queued; torch's allocator orders any reuse after it on this stream
    return o


def _op_forward_varlen(q, k, v, cu_seqlens, max_seqlen, params):
    """(o, lse [T, H]) through torch.ops.chia_attn.fwd_varlen."""
    from .library import call_fwd_varlen

    if not isinstance(q, torch.Tensor) or q.dim() != 3:
        raise ValueError("q must be a packed 3-D [T, heads, D] tensor")
    p = dict(params)
    H = q.shape[1]
    cache = (q.device.type == "cuda" and not torch.compiler.is_compiling()
             and not isinstance(q, torch._subclasses.fake_tensor.FakeTensor))
    p["head_scale"] = _per_head_vector(p["head_scale"], H, q.device, "head_scale", positive=True, cache=cache)
    p["alibi_slopes"] = _per_head_vector(p["alibi_slopes"], H, q.device, "alibi_slopes", positive=False,
                                         cache=cache)
    return call_fwd_varlen(q, k, v, cu_seqlens, max_seqlen, p)


def run_forward_varlen(q, k, v, cu_seqlens, max_seqlen, params):
    """(o, lse) for the registered operator: lse float32 [T, H] (softmax) or [0]."""
    T, H, _ = q.shape
    o = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)
    softmax = params["norm"] == "softmax"
    lse = torch.empty(T if softmax else 0, H if softmax else 0, dtype=torch.float32, device=q.device)
    if T == 0:
        check_cu_seqlens(cu_seqlens, 0, max_seqlen)
        return o, lse
    a, keep, qkv, _ = _prepare_varlen(q, k, v, cu_seqlens, max_seqlen, o, **params)
    with torch.cuda.device(q.device):
        _lib.fwd_lse(a, lse.data_ptr() if softmax else 0, torch.cuda.current_stream(q.device).cuda_stream)
    del keep, qkv  # queued: any reuse of their memory is ordered after the launch
    return o, lse


def run_backward_varlen(do, q, k, v, o, lse, cu_seqlens, max_seqlen, params):
    """dq, dk, dv of a packed batch by chia_attn_bwd."""
    dq, dk, dv = (torch.empty(t.shape, dtype=torch.bfloat16, device=t.device) for t in (q, k, v))
    if q.shape[0] == 0:
        return dq, dk, dv
    # keep (offsets, order, per-head vectors) and qkv (layout copies of q, k, v)
    # stay referenced until the launch is queued: do_ and the workspace are
    # allocated below and must not take their memory.
    a, keep, qkv, _ = _prepare_varlen(q, k, v, cu_seqlens, max_seqlen, o, **params)
    do_ = do if (do.dtype == torch.bfloat16 and _layout_ok_packed(do)) else do.to(torch.bfloat16).contiguous()
    if do_.shape != q.shape:
        raise ValueError(f"do must have q's shape {tuple(q.shape)}, got {tuple(do.shape)}")
    softmax = params["norm"] == "softmax"
    nbytes = _lib.bwd_workspace_size(a)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
    b = _lib.BwdArgs(dout=do_.data_ptr(), dq=dq.data_ptr(), dk=dk.data_ptr(), dv=dv.data_ptr(),
                     lse=lse.data_ptr() if softmax else None, workspace=ws.data_ptr(), workspace_bytes=nbytes)
    b.fwd = ctypes.pointer(a)
    for name, t in (("dout_stride", do_), ("dq_stride", dq), ("dk_stride", dk), ("dv_stride", dv)):
        st = getattr(b, name)
        st[0], st[1], st[2] = 0, t.stride(1), t.stride(0)
    with torch.cuda.device(q.device):
        _lib.bwd(b, torch.cuda.current_stream(q.device).cuda_stream)
    del keep, qkv, ws  # queued: any reuse of their memory is ordered after the launch
    return dq, dk, dv


def plan(*, batch: int, heads: int, seqlen: int, head_dim: int, **mask_kw) -> dict:
    """Host-only schedule statistics (tiles visited, exact visible pairs)."""
    return _lib.plan(make_args(batch=batch, heads=heads, seqlen=seqlen, head_dim=head_dim, **mask_kw))
