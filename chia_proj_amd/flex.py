"""FlexAttention-style front end: ``score_mod`` / ``mask_mod`` callables compiled to the core.

The reference compares its kernels with torch's FlexAttention, writing each
variant as a score modifier and a mask predicate (extra_bench.py:85-99):

    score_mod(score, b, h, q_idx, kv_idx) -> score'
    mask_mod(b, h, q_idx, kv_idx) -> bool

This module takes the same callables.  ``create_block_mask`` evaluates the
mask predicate on the index grid (row chunks, vectorised, on the requested
device) and compiles it to the core's mask parameters -- prefix, causal band,
window, dilation, block -- by fitting them from the evaluated mask and then
checking the fitted mask against the evaluated one on every (q_idx, kv_idx)
pair; the kernel then classifies its tiles from those parameters (the same
per-block key range and tile classes ``tile_map`` reports).  ``fit_score_mod``
probes the modifier numerically and fits
    score' = softcap * tanh((a_h * score + c_h * (kv_idx - q_idx)) / softcap) + offset
(softcap 0: no tanh): a per-head scale a_h (temperature), a per-head ALiBi
slope c_h and a softcap, checked at random points.  A predicate or modifier
outside these families raises ``NotExpressible``: nothing is approximated and
there is no fallback path.

Unlike FlexAttention, the sigmoid and ReLU normalisers (the reference's two
variants FlexAttention cannot express, extra_bench.py:100-103) are available
through ``norm=``.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Optional, Tuple

import torch

from . import _lib
from .attention import _op_forward, attention, make_args

MaskMod = Callable[..., torch.Tensor]
ScoreMod = Callable[..., torch.Tensor]

ROWS_PER_BLOCK = 128  # query rows of one block of the tile map (one 4-wavefront workgroup's block)
KEYS_PER_TILE = 64


class NotExpressible(ValueError):
    """The callable is outside the families the core implements."""


# ---------------------------------------------------------------- mask predicates

def _band_rows(rows: torch.Tensor, S: int, causal: bool, window: int, dilation: int, block: int,
               prefix: int) -> torch.Tensor:
    """The core's visibility predicate for query rows `rows` against keys 0..S-1."""
    i = rows.view(-1, 1)
    j = torch.arange(S, device=rows.device).view(1, -1)
    d = i - j
    ok = (d >= 0) if causal else torch.ones(1, S, dtype=torch.bool, device=rows.device)
    if window:
        ok = ok & ((d < window) if causal else (d.abs() < window))
    if dilation > 1:
        ok = ok & (torch.remainder(d, dilation) == 0)
    if block:
        ok = ok & (torch.div(i, block, rounding_mode="floor") == torch.div(j, block, rounding_mode="floor"))
    if prefix:
        ok = ok | (j < prefix)
    return ok.expand(rows.numel(), S)


def _eval_mask(mask_mod: MaskMod, b: int, h: int, rows: torch.Tensor, S: int) -> torch.Tensor:
    """mask_mod on the (rows x 0..S-1) grid as a bool [len(rows), S] tensor.  Tries a
    broadcast call first (index tensors [R, 1] and [1, S]), then vmap over both axes
    (the element-wise calling convention of FlexAttention)."""
    dev = rows.device
    bt = torch.tensor(b, device=dev)
    ht = torch.tensor(h, device=dev)
    qi = rows.view(-1, 1)
    kj = torch.arange(S, device=dev).view(1, -1)
    try:
        m = mask_mod(bt, ht, qi, kj)
        m = torch.as_tensor(m, device=dev)
        m = m.to(torch.bool).expand(rows.numel(), S)
    except Exception:  # noqa: BLE001 -- element-wise predicates (data-dependent Python control flow)
        inner = torch.vmap(lambda q, k: mask_mod(bt, ht, q, k), in_dims=(None, 0))
        m = torch.vmap(inner, in_dims=(0, None))(rows, torch.arange(S, device=dev)).to(torch.bool)
    return m


def _row_chunks(S: int, device) -> list:
    step = max(1, (1 << 24) // max(S, 1))
    return [torch.arange(r0, min(S, r0 + step), device=device) for r0 in range(0, S, step)]


@dataclass(frozen=True)
class BlockMask:
    """A mask predicate compiled to the core's mask parameters for sequence length
    ``seq_len`` (queries and keys).  ``mask_kwargs()`` are attention()'s keyword
    arguments; ``tile_map()`` and the FlexAttention-named properties give the
    per-block key ranges and tile classes the kernel derives from them."""
    seq_len: int
    causal: bool
    window: int
    dilation: int
    block: int
    prefix: int
    BLOCK_SIZE: Tuple[int, int] = (ROWS_PER_BLOCK, KEYS_PER_TILE)

    def mask_kwargs(self) -> dict:
        return dict(causal=self.causal, window=self.window, dilation=self.dilation, block=self.block,
                    prefix=self.prefix)

    def to_dense(self, device="cpu") -> torch.Tensor:
        """bool [S, S]: query i sees key j."""
        rows = torch.arange(self.seq_len, device=device)
        return _band_rows(rows, self.seq_len, **self.mask_kwargs()).clone()

    def tile_map(self, residue: int = 0):
        """int8 [query blocks, key tiles] of residue class `residue` (sub-sequence
        coordinates; one class unless dilation > 1): 0 empty, 1 full, 2 partial."""
        a = make_args(batch=1, heads=1, seqlen=self.seq_len, head_dim=64, **self.mask_kwargs())
        return _lib.tile_map(a, residue, ROWS_PER_BLOCK)

    def _indices(self, cls):
        tm = torch.from_numpy(self.tile_map(0).astype("int64"))
        sel = (tm == 1) if cls == "full" else (tm == 2)
        num = sel.sum(1).to(torch.int32)
        idx = torch.zeros(tm.shape, dtype=torch.int32)
        for qb in range(tm.shape[0]):
            nz = torch.nonzero(sel[qb]).flatten()
            idx[qb, :nz.numel()] = nz.to(torch.int32)
        return num, idx

    @property
    def kv_num_blocks(self):
        """Partial key tiles per query block (FlexAttention's name; residue 0)."""
        return self._indices("partial")[0]

    @property
    def kv_indices(self):
        return self._indices("partial")[1]

    @property
    def full_kv_num_blocks(self):
        return self._indices("full")[0]

    @property
    def full_kv_indices(self):
        return self._indices("full")[1]


def _band_stats(chunks, evals, S: int, P: int):
    """Over visible pairs with key >= P: min and max of d = i - j and the smallest
    nonzero |d| (None when there is no such pair)."""
    dmin, dmax, dpos = None, None, None
    j = None
    for rows, m in zip(chunks, evals()):
        if j is None or j.device != rows.device:
            j = torch.arange(S, device=rows.device).view(1, -1)
        d = rows.view(-1, 1) - j
        sel = m & (j >= P)
        if not sel.any():
            continue
        dv = d[sel]
        lo, hi = int(dv.min()), int(dv.max())
        dmin = lo if dmin is None else min(dmin, lo)
        dmax = hi if dmax is None else max(dmax, hi)
        nz = dv.abs()[dv != 0]
        if nz.numel():
            p = int(nz.min())
            dpos = p if dpos is None else min(dpos, p)
    return dmin, dmax, dpos


def _first_violation(chunks, evals, S: int, params: dict):
    """The first (row, key) pair, in row order and nearest the diagonal within the
    row, that the band without a block predicts visible but the mask hides."""
    for rows, m in zip(chunks, evals()):
        v = _band_rows(rows, S, **params) & ~m
        if v.any():
            r = int(torch.nonzero(v.any(1)).flatten()[0])
            i = int(rows[r])
            js = torch.nonzero(v[r]).flatten()
            j = int(js[torch.argmin((js - i).abs())])
            return i, j
    return None


def _divisors(n: int) -> set:
    out = set()
    x = 1
    while x * x <= n:
        if n % x == 0:
            out.update((x, n // x))
        x += 1
    return out


def _matches(chunks, evals, S: int, params: dict) -> bool:
    return all(torch.equal(_band_rows(rows, S, **params), m) for rows, m in zip(chunks, evals()))


def create_block_mask(mask_mod: MaskMod, B: Optional[int], H: Optional[int], Q_LEN: int, KV_LEN: int,
                      device="cpu", check_rows: int = 64) -> BlockMask:
    """Compile `mask_mod` for sequence length Q_LEN == KV_LEN.

    The predicate is evaluated for (b, h) = (0, 0) on every pair; when B or H is
    given it is also evaluated on `check_rows` spread rows for other (b, h)
    values and must not depend on them (the core's masks are the same for every
    batch and head).  Raises NotExpressible when no parameter set of the core
    reproduces the evaluated mask exactly."""
    if Q_LEN != KV_LEN:
        raise NotExpressible(f"the core is self-attention: Q_LEN must equal KV_LEN, got {Q_LEN}, {KV_LEN}")
    S = int(Q_LEN)
    if S < 1:
        raise ValueError("Q_LEN must be >= 1")
    device = torch.device(device)
    chunks = _row_chunks(S, device)
    cached = [] if S * S <= (1 << 27) else None
    if cached is not None:
        cached.extend(_eval_mask(mask_mod, 0, 0, rows, S) for rows in chunks)

    def evals():
        if cached is not None:
            return iter(cached)
        return (_eval_mask(mask_mod, 0, 0, rows, S) for rows in chunks)

    # batch / head independence on spread rows
    nb, nh = (B or 1), (H or 1)
    if nb * nh > 1:
        probe = torch.unique(torch.linspace(0, S - 1, min(S, check_rows), device=device).round().long())
        ref = _eval_mask(mask_mod, 0, 0, probe, S)
        pairs = {(b, h) for b in (0, nb - 1, nb // 2) for h in (0, nh - 1, nh // 2)} - {(0, 0)}
        for b, h in sorted(pairs):
            if not torch.equal(_eval_mask(mask_mod, b, h, probe, S), ref):
                raise NotExpressible(f"mask_mod depends on the batch or head index ((b, h) = {(b, h)} differs "
                                     "from (0, 0)); the core's masks are shared by all batches and heads")

    # leading keys every query sees: a candidate prefix
    col_all = None
    for m in evals():
        c = m.all(0)
        col_all = c if col_all is None else (col_all & c)
    lead = int(torch.cumprod(col_all.to(torch.int64), 0).sum())
    if lead == S:
        return BlockMask(S, False, 0, 1, 0, 0)

    for P in dict.fromkeys((0, lead)):
        dmin, dmax, dpos = _band_stats(chunks, evals, S, P)
        if dmin is None:  # nothing visible beyond the prefix
            cands = [dict(causal=True, window=1, dilation=1, block=0, prefix=P)] if P else []
        else:
            causal = dmin >= 0
            dil = dpos if dpos is not None else 1
            reach = dmax if causal else max(dmax, -dmin)
            # no window when no farther pair (a multiple of dil, key >= P) exists;
            # otherwise the largest equivalent window (the next multiple of dil)
            limit = S - 1 - P if causal else S - 1
            window = 0 if reach + dil > limit else reach + dil
            base = dict(causal=causal, window=window, dilation=dil, block=0, prefix=P)
            cands = [base]
            v = _first_violation(chunks, evals, S, base)
            if v is not None:
                # a pair the band allows but the mask hides straddles a block
                # boundary: some multiple of the block lies in (min(i, j), max(i, j)]
                # (earlier boundaries may hide under the prefix); candidates pass a
                # check on spread rows before the full one, and a block may make the
                # window redundant
                i, j = v
                blks = set()
                for beta in range(min(i, j) + 1, max(i, j) + 1):
                    blks.update(_divisors(beta))
                probe = torch.unique(torch.cat([
                    torch.linspace(0, S - 1, min(S, 128), device=device).round().long(),
                    torch.tensor([i, j, min(i, j) + 1, max(i, j) - 1], device=device).clamp(0, S - 1)]))
                pm = _eval_mask(mask_mod, 0, 0, probe, S)
                for blk in sorted(blks, reverse=True):
                    for c in (dict(base, block=blk, window=0), dict(base, block=blk)):
                        if torch.equal(_band_rows(probe, S, **c), pm):
                            cands.append(c)
        for c in cands:
            if c["dilation"] > 1 and c["prefix"] > 0:
                continue  # not a combination the core implements
            if _matches(chunks, evals, S, c):
                return BlockMask(S, c["causal"], c["window"], c["dilation"], c["block"], c["prefix"])
    raise NotExpressible("mask_mod is not a prefix / causal-band / window / dilation / block-diagonal mask "
                         "the core implements (checked against every (q_idx, kv_idx) pair)")


# ---------------------------------------------------------------- score modifiers

@dataclass(frozen=True)
class FittedScoreMod:
    """score' = softcap * tanh((head_scale[h] * s + alibi_slopes[h] * (kv - q)) / softcap) + offset."""
    heads: int
    head_scale: Optional[Tuple[float, ...]]
    alibi_slopes: Optional[Tuple[float, ...]]
    softcap: float
    offset: float


def _call_score(score_mod: ScoreMod, s, b, h, qi, kj):
    try:
        out = score_mod(s, b, h, qi, kj)
    except Exception:  # noqa: BLE001 -- element-wise modifiers
        out = torch.vmap(score_mod)(s, b, h, qi, kj)
    return torch.as_tensor(out, device=s.device).to(torch.float64).expand(s.shape)


def fit_score_mod(score_mod: ScoreMod, heads: int, seq_len: int, batch: int = 1, device="cpu",
                  probes: int = 4096, seed: int = 0, rtol: float = 2e-5) -> FittedScoreMod:
    """Fit `score_mod` to the core's modifier family (see the module docstring) and
    check it at `probes` random (score, b, h, q_idx, kv_idx) points, |error| <=
    rtol * (1 + |score'|).  Raises NotExpressible otherwise."""
    dev = torch.device(device)
    H = int(heads)
    hs = torch.arange(H, device=dev)
    z = torch.zeros(H, dtype=torch.long, device=dev)

    def f(s, h, qi, kj, b=None):
        s = torch.as_tensor(s, dtype=torch.float64, device=dev).expand(h.shape)
        return _call_score(score_mod, s.clone(), z[:1].expand(h.shape) if b is None else b, h, qi, kj)

    f0 = f(0.0, hs, z, z)
    offset = float(f0[0])
    if not torch.allclose(f0, torch.full_like(f0, offset), rtol=0, atol=1e-12):
        raise NotExpressible("score_mod(0) differs between heads: a per-head additive constant is not supported")
    big = f(1e6, hs, z, z) - offset
    neg = f(-1e6, hs, z, z) - offset
    capped = bool((big.abs() < 1e5).all())
    cap = float(big[0]) if capped else 0.0
    if capped and not (cap > 0 and torch.allclose(big, torch.full_like(big, cap), rtol=1e-6)
                       and torch.allclose(neg, torch.full_like(neg, -cap), rtol=1e-6)):
        raise NotExpressible("score_mod is bounded but not a symmetric per-call softcap")

    def lin(x):  # the pre-cap value behind an output x (offset removed)
        if not capped:
            return x
        y = (x / cap).clamp(-1 + 1e-15, 1 - 1e-15)
        return cap * torch.atanh(y)

    s1 = 1e-3 * cap if capped else 1.0
    a = (lin(f(s1, hs, z, z) - offset) - lin(f(-s1, hs, z, z) - offset)) / (2 * s1)
    one = torch.ones_like(z)
    c = lin(f(0.0, hs, z, one) - offset)

    g = torch.Generator("cpu").manual_seed(seed)
    n = int(probes)
    span = 4.0 * (cap if capped else 10.0)
    s = ((torch.rand(n, generator=g, dtype=torch.float64) * 2 - 1) * span).to(dev)
    hh = torch.randint(0, H, (n,), generator=g).to(dev)
    bb = torch.randint(0, max(1, int(batch)), (n,), generator=g).to(dev)
    qi = torch.randint(0, max(1, int(seq_len)), (n,), generator=g).to(dev)
    kj = torch.randint(0, max(1, int(seq_len)), (n,), generator=g).to(dev)
    got = _call_score(score_mod, s.clone(), bb, hh, qi, kj)
    u = a[hh] * s + c[hh] * (kj - qi).to(torch.float64)
    want = (cap * torch.tanh(u / cap) if capped else u) + offset
    err = ((got - want).abs() / (1 + want.abs())).max().item()
    if not err <= rtol:
        raise NotExpressible(f"score_mod is not scale * score + slope * (kv_idx - q_idx) (optionally softcapped): "
                             f"max relative misfit {err:.3g} at random probes")
    if not bool((a > 0).all()):
        raise NotExpressible("score_mod's per-head scale must be > 0")
    a_t = tuple(float(x) for x in a.cpu())
    c_t = tuple(float(x) for x in c.cpu())
    # the kernel takes float32 constants: unit scales and zero slopes drop out
    unit = bool((a.to(torch.float32) == 1.0).all())
    flat = bool((c.to(torch.float32) == 0.0).all())
    return FittedScoreMod(H, None if unit else a_t, None if flat else c_t, cap, offset)


# ---------------------------------------------------------------- entry point

def flex_params(query_shape, score_mod=None, block_mask: Optional[BlockMask] = None, scale: Optional[float] = None,
                *, norm: str = "softmax", bias: float = 0.0, post_scale: float = 1.0, device="cpu"):
    """attention()'s keyword arguments for a flex_attention call on a [B, H, S, D]
    query, and the fitted score modifier (None without one)."""
    B, H, S, _ = query_shape
    if block_mask is None:
        mask = dict(causal=False, window=0, dilation=1, block=0, prefix=0)
    else:
        if block_mask.seq_len != S:
            raise ValueError(f"block_mask was built for length {block_mask.seq_len}, the inputs have {S}")
        mask = block_mask.mask_kwargs()
    fitted = score_mod
    if score_mod is not None and not isinstance(score_mod, FittedScoreMod):
        # probe on the host unless the modifier's captured tensors live on the device
        try:
            fitted = fit_score_mod(score_mod, H, S, batch=B, device="cpu")
        except NotExpressible:
            raise
        except RuntimeError:
            fitted = fit_score_mod(score_mod, H, S, batch=B, device=device)
    params = dict(norm=norm, scale=scale, head_scale=None, alibi_slopes=None, softcap=0.0, bias=bias,
                  post_scale=post_scale, **mask)
    if fitted is not None:
        if fitted.heads != H:
            raise ValueError(f"score_mod was fitted for {fitted.heads} heads, the query has {H}")
        if fitted.offset and norm == "relu":
            raise NotExpressible("an additive constant in score_mod changes relu(score) and is not supported")
        if norm == "sigmoid":
            params["bias"] = bias + fitted.offset
        # softmax: a constant added to every score cancels
        params.update(head_scale=fitted.head_scale and list(fitted.head_scale),
                      alibi_slopes=fitted.alibi_slopes and list(fitted.alibi_slopes), softcap=fitted.softcap)
    return params, fitted


def flex_attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, score_mod=None,
                   block_mask: Optional[BlockMask] = None, scale: Optional[float] = None, enable_gqa: bool = False,
                   return_lse: bool = False, *, norm: str = "softmax", bias: float = 0.0, post_scale: float = 1.0):
    """torch.nn.attention.flex_attention's call on the gfx950 core.

    query [B, H, S, D], key / value [B, H_kv, S, D] bf16 on the GPU (H_kv < H needs
    enable_gqa).  block_mask None is full (non-causal) attention.  score_mod is a
    callable (fitted at every call) or a FittedScoreMod.  norm "sigmoid" applies
    sigmoid(score' + bias) * post_scale, "relu" relu(score') * post_scale.
    Returns o, or (o, lse) with lse float32 [B, H, S] (softmax only).
    """
    if key.shape[1] != query.shape[1] and not enable_gqa:
        raise ValueError("key has fewer heads than query: pass enable_gqa=True")
    params, fitted = flex_params(tuple(query.shape), score_mod, block_mask, scale, norm=norm, bias=bias,
                                 post_scale=post_scale, device=query.device)
    if return_lse:
        if norm != "softmax":
            raise ValueError("return_lse needs norm='softmax'")
        o, lse = _op_forward(query, key, value, params)
        # a constant added to every score leaves o unchanged and shifts lse by it
        return o, (lse + fitted.offset if fitted is not None and fitted.offset else lse)
    return attention(query, key, value, **params)
