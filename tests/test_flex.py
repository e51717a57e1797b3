"""The FlexAttention-style front end (chia_proj_amd/flex.py) without a GPU.

Pins: the reference's own FlexAttention descriptions of its variants
(extra_bench.py:86-95, restated below as predicates and modifiers) compile to
the parameters of this library's hand-written variants; compiled masks equal
the oracle's mask (oracle.generic.visible_mask, an independent formula) on
every pair for random parameter sets; tile metadata agrees with the dense
mask; predicates and modifiers outside the core's families are refused."""
import itertools
import random

import numpy as np
import pytest
import torch

from chia_proj_amd import core_kwargs
from chia_proj_amd.flex import (BlockMask, FittedScoreMod, NotExpressible, create_block_mask, fit_score_mod,
                                flex_params)
from oracle.generic import visible_mask

from flex_cases import FLEX_REF, H_REF, SLOPES, TEMPS, causal

S_REF = 2048
MASK_KEYS = ("causal", "window", "dilation", "block", "prefix")


def _canon(kw):
    out = dict(causal=bool(kw.get("causal", True)), window=int(kw.get("window") or 0),
               dilation=int(kw.get("dilation") or 1), block=int(kw.get("block") or 0),
               prefix=int(kw.get("prefix") or 0))
    return out


@pytest.mark.parametrize("op,score_mod,mask_mod", FLEX_REF, ids=[r[0] for r in FLEX_REF])
def test_reference_flex_descriptions_compile_to_the_variants(op, score_mod, mask_mod):
    bm = create_block_mask(mask_mod, None, None, S_REF, S_REF)
    params, fitted = flex_params((4, H_REF, S_REF, 64), score_mod, bm)
    want = core_kwargs(op, H_REF)
    if op == "temp_perhead":
        want["head_scale"] = TEMPS  # FlexAttention's temperatures are float32, the eager path's bf16
    assert {k: params[k] for k in MASK_KEYS} == _canon(want)
    for key in ("head_scale", "alibi_slopes"):
        if want.get(key) is None:
            assert params[key] is None, key
        else:
            np.testing.assert_allclose(np.asarray(params[key], dtype=np.float32),
                                       torch.as_tensor(want[key], dtype=torch.float32).numpy(), rtol=1e-7)
    assert params["softcap"] == float(want.get("softcap", 0.0))
    assert torch.equal(bm.to_dense(), visible_mask(S_REF, **_canon(want)))


def _random_masks(n, seed):
    rng = random.Random(seed)
    out = []
    while len(out) < n:
        S = rng.choice([1, 2, 5, 63, 64, 65, 127, 200, 333])
        kw = dict(causal=rng.random() < 0.6, window=rng.choice([0, 0, 1, 2, 7, 50, 130]),
                  dilation=rng.choice([1, 1, 2, 3, 5]), block=rng.choice([0, 0, 1, 16, 37, 100]),
                  prefix=rng.choice([0, 0, 3, 40]))
        if kw["dilation"] > 1 and kw["prefix"]:
            continue
        if not visible_mask(S, **kw).any():
            continue  # an empty mask is not expressible
        out.append((S, kw))
    return out


@pytest.mark.parametrize("S,kw", _random_masks(60, 7), ids=[f"{s}-{k}" for s, k in _random_masks(60, 7)])
def test_compiled_mask_equals_oracle_mask(S, kw):
    want = visible_mask(S, **kw)
    bm = create_block_mask(lambda b, h, q, k: visible_mask(S, **kw)[q, k], 2, 3, S, S)
    assert torch.equal(bm.to_dense(), want), (bm, kw)


def test_element_wise_predicate_uses_vmap():
    # stack() needs equal shapes: fails on the broadcast grid, works element-wise
    def diag_band(b, h, q, k):
        d = torch.stack([q, k]).diff(dim=0).squeeze(0)  # k - q
        return (d <= 0) & (d > -10)

    bm = create_block_mask(diag_band, None, None, 100, 100)
    assert bm.mask_kwargs() == dict(causal=True, window=10, dilation=1, block=0, prefix=0)


@pytest.mark.parametrize("name,mask_mod", [
    ("two_bands", lambda b, h, q, k: ((q - k).abs() < 3) | ((q - k).abs() == 20)),
    ("anti_causal_window", lambda b, h, q, k: (k >= q) & (k - q < 5) & (q > 3)),
    ("products", lambda b, h, q, k: (q * k) % 3 == 0),
    ("nothing", lambda b, h, q, k: q < 0),
])
def test_inexpressible_masks_are_refused(name, mask_mod):
    with pytest.raises(NotExpressible):
        create_block_mask(mask_mod, None, None, 96, 96)


def test_head_dependent_mask_is_refused():
    with pytest.raises(NotExpressible, match="batch or head"):
        create_block_mask(lambda b, h, q, k: (k <= q) | (h == 3), 1, 4, 128, 128)
    with pytest.raises(NotExpressible, match="Q_LEN"):
        create_block_mask(causal, None, None, 128, 256)


@pytest.mark.parametrize("kw", [dict(causal=True), dict(causal=True, window=300), dict(causal=False, block=200),
                                dict(causal=True, prefix=130), dict(causal=True, dilation=2, window=500)])
def test_tile_metadata_agrees_with_dense_mask(kw, lib_built):
    S = 700
    bm = BlockMask(S, **_canon(kw))
    dense = bm.to_dense().numpy()
    sub = dense[0::bm.dilation, 0::bm.dilation]  # residue class 0
    full_n, full_i = bm.full_kv_num_blocks, bm.full_kv_indices
    part_n, part_i = bm.kv_num_blocks, bm.kv_indices
    rows, keys = bm.BLOCK_SIZE
    for qb in range(full_n.numel()):
        tiles = {int(t): "full" for t in full_i[qb, :full_n[qb]]}
        tiles.update({int(t): "partial" for t in part_i[qb, :part_n[qb]]})
        for kt in range((sub.shape[1] + keys - 1) // keys):
            blk = sub[qb * rows:(qb + 1) * rows, kt * keys:(kt + 1) * keys]
            cls = tiles.get(kt, "empty")
            if cls == "full":
                assert blk.shape[1] == keys and blk.all()
            elif cls == "empty":
                assert not blk.any()


def test_score_mod_fits():
    f = fit_score_mod(lambda s, b, h, q, k: torch.tanh((s * TEMPS[h] + SLOPES[h] * 0.01 * (k - q)) / 7.0) * 7.0,
                      H_REF, 4096, batch=3)
    assert f.softcap == pytest.approx(7.0, rel=1e-12)
    np.testing.assert_allclose(f.head_scale, TEMPS.double().numpy(), rtol=1e-9)
    np.testing.assert_allclose(f.alibi_slopes, (SLOPES * 0.01).double().numpy(), rtol=1e-9)  # float32 product
    f = fit_score_mod(lambda s, b, h, q, k: s / TEMPS[h], H_REF, 512)
    np.testing.assert_allclose(f.head_scale, (1.0 / TEMPS.double()).numpy(), rtol=1e-6)
    f = fit_score_mod(lambda s, b, h, q, k: s, 4, 64)
    assert f == FittedScoreMod(4, None, None, 0.0, 0.0)


@pytest.mark.parametrize("name,score_mod", [
    ("square", lambda s, b, h, q, k: s * s),
    ("relative_product", lambda s, b, h, q, k: s * (k - q)),
    ("head_offset", lambda s, b, h, q, k: s + h),
    ("negative_scale", lambda s, b, h, q, k: -s),
    ("batch_dependent", lambda s, b, h, q, k: s * (b + 1)),
    ("asymmetric_cap", lambda s, b, h, q, k: torch.clamp(s, -3.0, 5.0)),
    ("quadratic_position", lambda s, b, h, q, k: s - 0.001 * (k - q) ** 2),
])
def test_inexpressible_score_mods_are_refused(name, score_mod):
    with pytest.raises(NotExpressible):
        fit_score_mod(score_mod, 4, 300, batch=2)


def test_offsets_map_per_normaliser():
    shape = (1, 4, 64, 64)
    params, _ = flex_params(shape, lambda s, b, h, q, k: s + 2.5, norm="sigmoid", bias=-1.0)
    assert params["bias"] == pytest.approx(1.5) and params["norm"] == "sigmoid"
    params, _ = flex_params(shape, lambda s, b, h, q, k: s + 2.5)  # softmax: cancels
    assert params["bias"] == 0.0 and params["head_scale"] is None
    with pytest.raises(NotExpressible):
        flex_params(shape, lambda s, b, h, q, k: s + 2.5, norm="relu")
    params, _ = flex_params(shape, None, None)  # no block mask: full attention
    assert {k: params[k] for k in MASK_KEYS} == dict(causal=False, window=0, dilation=1, block=0, prefix=0)
