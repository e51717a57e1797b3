"""GPU parity: the HIP core (through the C ABI) against the CPU oracle.

Gate: bf16 output vs the fp32 oracle within max-abs 2e-2 and mean-abs 2e-3
(GATE_MAX_ABS / GATE_MEAN_ABS in chia_proj_amd.gate), plus the reference's
own gate (synth10.py:173-184: rel < 3e-2 at input scales 1.0 and 0.01).
Full-size cases run the kernel over the whole shape, check that every output
is finite, and gate every (batch, head) slice against the oracle (computed a
batch at a time), as the reference gates its whole output tensor
(extra_bench.py:29,121; shape_gen.py:97-110).
"""
import math

import pytest
import torch

import oracle
from chia_proj_amd import OPS, attention, gate
from chia_proj_amd.workloads import baseline_configs, draw_inputs, suite

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _say(msg):
    print(msg, flush=True)


def _unnormalised(op, params):
    """sigmoid / ReLU without the BASELINE's -log S or 1/S factor: output grows like sqrt(S)."""
    if op == "sigmoid_attn":
        return params.get("bias", 0.0) > -1.0
    if op == "relu_attn":
        return params.get("post_scale", 1.0) > 0.1
    return False


def _check_case(op, q, k, v, params, heads=None):
    """Run variant `op` on the whole shape; gate `heads` ((b, h) pairs) against the
    oracle, or every slice when heads is None (the oracle runs a batch at a time)."""
    o = OPS[op](q, k, v, **params)
    torch.cuda.synchronize()
    assert o.shape == q.shape and o.dtype == torch.bfloat16
    assert bool(torch.isfinite(o).all()), f"{op}: non-finite output"
    B, H = q.shape[:2]
    qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
    oc = o.float().cpu()
    unnorm = _unnormalised(op, params)
    if heads is not None:
        refs = oracle.variant_ref_heads(op, qc, kc, vc, heads, **params)
        for (b, h), r in zip(heads, refs):
            res = gate.north_star_gate(r, oc[b, h], scale_aware=unnorm)
            assert res.ok, f"{op} b={b} h={h}: {res.status} {res.stats}"
        return
    worst = (0.0, 0.0)
    for b in range(B):
        # variant_ref resolves the per-head parameters for the batch's H heads itself
        ref = oracle.variant_ref(op, qc[b:b + 1], kc[b:b + 1], vc[b:b + 1], **params)
        for h in range(H):
            res = gate.north_star_gate(ref[0, h], oc[b, h], scale_aware=unnorm)
            assert res.ok, f"{op} b={b} h={h}: {res.status} {res.stats}"
            worst = max(worst, (res.stats["max_abs"], res.stats["mean_abs"]))
    _say(f"  {op}: {B * H} slices within the gate, worst max-abs {worst[0]:.3e}")


@pytest.mark.parametrize("op", list(OPS))
@pytest.mark.parametrize("D", [64, 128])
def test_reference_defaults_small(op, D):
    """Every variant with the reference's constants at B1 H4 S1024."""
    _say(f"[parity] defaults op={op} D={D}")
    g = torch.Generator("cpu").manual_seed(1000 + D)
    q, k, v = (torch.randn(1, 4, 1024, D, generator=g).to(torch.bfloat16).to(DEV) for _ in range(3))
    _check_case(op, q, k, v, {}, heads=[(0, h) for h in range(4)])


@pytest.mark.parametrize("case", baseline_configs(), ids=lambda c: c.name)
def test_baseline_configs(case):
    """The five BASELINE.json configurations at full size, every (batch, head) slice."""
    _say(f"[parity] config {case.name}")
    q, k, v, params = draw_inputs(case, DEV)
    _check_case(case.op, q, k, v, params)


@pytest.mark.parametrize("op", list(OPS))
@pytest.mark.parametrize("S", [1024, 2048, 4096])
def test_north_star_sweep(S, op):
    """Each of the ten variants, BASELINE parameters, B4 H16 D64, S in {1024, 2048,
    4096} (4096: the north-star shape), every (batch, head) slice."""
    case = next(c for c in suite(4, 16, S, 64) if c.op == op)
    _say(f"[parity] sweep {case.name} S={S}")
    q, k, v, params = draw_inputs(case, DEV)
    _check_case(case.op, q, k, v, params)


@pytest.mark.parametrize("op", list(OPS))
def test_reference_gate_scales(op):
    """The reference's verify() at input scales 1.0 and 0.01 (synth10.py:173-184)."""
    _say(f"[parity] reference gate op={op}")
    g = torch.Generator("cpu").manual_seed(77)
    q, k, v = (torch.randn(1, 2, 512, 128, generator=g).to(torch.bfloat16).to(DEV) for _ in range(3))
    ok, worst, msg = gate.verify(lambda a, b, c: OPS[op](a, b, c).float().cpu(),
                                 lambda a, b, c: oracle.variant_ref(op, a.cpu(), b.cpu(), c.cpu()), q, k, v)
    assert ok, f"{op}: {msg}"


EDGE = [
    # (name, S, D, generic kwargs)
    ("S1_causal", 1, 64, dict(causal=True)),
    ("S7_full", 7, 64, dict(causal=False)),
    ("S65_causal", 65, 128, dict(causal=True)),
    ("S100_window17", 100, 64, dict(causal=True, window=17)),
    ("S257_local40", 257, 64, dict(causal=False, window=40)),
    ("S1000_dil3", 1000, 64, dict(causal=True, dilation=3)),
    ("S999_dil5_w300", 999, 128, dict(causal=True, dilation=5, window=300)),
    ("S777_block100", 777, 64, dict(causal=True, block=100)),
    ("S777_block100_full", 777, 64, dict(causal=False, block=100)),
    ("S600_prefix130", 600, 64, dict(causal=True, prefix=130)),
    ("S300_prefix_ge_S", 300, 64, dict(causal=True, prefix=1000)),
    ("S300_window_ge_S", 300, 64, dict(causal=True, window=5000)),
    ("S300_block_ge_S", 300, 64, dict(causal=True, block=4096)),
    ("S513_dil2_block64", 513, 64, dict(causal=True, dilation=2, block=64)),
    ("S640_sigmoid_win", 640, 64, dict(norm="sigmoid", causal=True, window=100, bias=-1.5)),
    ("S640_relu_local", 640, 128, dict(norm="relu", causal=False, window=70, post_scale=0.01)),
    ("S512_softcap_window", 512, 64, dict(causal=True, window=128, softcap=20.0)),
    ("S512_alibi_dil", 512, 64, dict(causal=True, dilation=2, alibi_slopes=[0.5, 0.25])),
    ("S512_sigmoid_softcap_alibi", 512, 128, dict(norm="sigmoid", causal=False, softcap=10.0,
                                                   alibi_slopes=[0.01, 0.02], bias=0.3)),
    ("S384_relu_softcap", 384, 64, dict(norm="relu", causal=True, softcap=5.0, post_scale=0.1)),
    ("S384_headscale", 384, 64, dict(causal=True, head_scale=[0.5, 2.0])),
    ("S384_noncausal_block_band", 384, 64, dict(causal=False, block=32, window=3)),
    # plain sigmoid takes the bias as the factor 2^(-bias log2 e): near the end of
    # that range (|bias log2 e| = 115), and past it (137: the general score path)
    ("S640_sigmoid_bias_fold_limit", 640, 64, dict(norm="sigmoid", causal=False, scale=10.0, bias=-80.0)),
    ("S640_sigmoid_bias_general", 640, 64, dict(norm="sigmoid", causal=True, scale=12.0, bias=-95.0)),
    ("S640_sigmoid_bias_general_pos", 640, 128, dict(norm="sigmoid", causal=False, scale=12.0, bias=95.0)),
]


# Scale-aware tolerances (relative to max|ref|) of edge cases outside the
# default ones.  Score scale 10: the plain sigmoid kernel takes Q pre-scaled by
# -scale log2 e and rounded to bf16, a relative error of 2^-9 on exponents of
# magnitude ~100 (measured 1.2e-2 and 1.3e-3 of max|ref|).
EDGE_SCALED = {"S640_sigmoid_bias_fold_limit": (2e-2, 2e-3)}


@pytest.mark.parametrize("name,S,D,kw", EDGE, ids=[e[0] for e in EDGE])
def test_edge_cases(name, S, D, kw):
    """Ragged lengths, combined masks and modifiers through the generic entry point."""
    _say(f"[parity] edge {name}")
    g = torch.Generator("cpu").manual_seed(S * 7 + D)
    q, k, v = (torch.randn(1, 2, S, D, generator=g).to(torch.bfloat16) for _ in range(3))
    o = attention(q.to(DEV), k.to(DEV), v.to(DEV), **kw)
    torch.cuda.synchronize()
    r = oracle.attention_ref(q, k, v, **kw)
    sm, sn = EDGE_SCALED.get(name, (gate.SCALED_MAX_ABS, gate.SCALED_MEAN_ABS))
    res = gate.north_star_gate(r, o.float().cpu(), scale_aware=kw.get("norm", "softmax") != "softmax",
                               scaled_max_abs=sm, scaled_mean_abs=sn)
    assert res.ok, f"{name}: {res.status} {res.stats}"


RISING = [
    ("causal", dict(causal=True)),
    ("prefix256", dict(causal=True, prefix=256)),
    ("full", dict(causal=False)),
    ("softcap50", dict(causal=True, softcap=50.0)),
    ("headscale", dict(causal=True, head_scale="per-head")),
    ("window256", dict(causal=True, window=256)),
    ("block256", dict(causal=False, block=256)),
    ("window200_softcap30", dict(causal=True, window=200, softcap=30.0)),
    ("local100_dil2", dict(causal=False, window=100, dilation=2)),
    ("softcap80", dict(causal=True, softcap=80.0)),  # above the fixed-reference limit: the running max
]


ALIBI_ORDER = [
    ("causal", dict(causal=True), 1.0),
    ("full", dict(causal=False), 1.0),
    ("prefix300", dict(causal=True, prefix=300), 1.0),
    ("causal_negative", dict(causal=True), -1.0),
    ("full_negative", dict(causal=False), -1.0),
    ("window300", dict(causal=True, window=300), 1.0),
    ("block256_negative", dict(causal=False, block=256), -1.0),
]


# Which core runs these shapes at head dim 64: B1 H2 (two slices) the paired core
# on 2-wavefront workgroups; B4 H16 S2048 the paired core on 4-wavefront ones
# (PAIR, WIDE and WIDE2 steps) for full rows, the one-block core for causal
# softmax, prefixes, windows and blocks; B2 H16 S4096 (32 slices) the paired core
# on 4-wavefront workgroups for causal rows too.  Head dim 128 runs the
# one-block core throughout.
PAIRED_CAUSAL = (2, 16, 4096)


def _alibi_order_case(name, kw, sign, shape, D):
    B, H, S = shape
    _say(f"[parity] alibi tile order {name} {shape} D{D}")
    g = torch.Generator("cpu").manual_seed(S + 3 * len(name) + D)
    q, k, v = (torch.randn(B, H, S, D, generator=g).to(torch.bfloat16) for _ in range(3))
    slopes = [sign * 2.0 * 0.5 ** h for h in range(H)]
    o = attention(q.to(DEV), k.to(DEV), v.to(DEV), alibi_slopes=slopes, **kw)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(o).all()), f"{name}: non-finite output"
    oc = o.float().cpu()
    for b, h in {(0, 0), (0, H - 1), (B - 1, H // 2), (B // 2, 1 % H)}:
        r = oracle.attention_ref(q[b:b + 1, h:h + 1], k[b:b + 1, h:h + 1], v[b:b + 1, h:h + 1],
                                 alibi_slopes=[slopes[h]], **kw)
        res = gate.north_star_gate(r[0, 0], oc[b, h])
        assert res.ok, f"{name} b={b} h={h}: {res.status} {res.stats}"


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("shape", [(1, 2, 700), (4, 16, 2048)], ids=["B1H2S700", "B4H16S2048"])
@pytest.mark.parametrize("name,kw,sign", ALIBI_ORDER, ids=[a[0] for a in ALIBI_ORDER])
def test_alibi_softmax_tile_order(name, kw, sign, shape, D):
    """ALiBi softmax walks the key tiles from the last to the first (both cores), with the row
    max only on demand (paired core, one-block core at head dim 64).  Steep slopes (up to 2 per
    key) with the standard sign put a row's max on its first tile; the negated slopes put it on
    the last one, so the exact fallback (or, in the one-block core at head dim 128, the rescale)
    runs on almost every tile.  Prefix tiles come after the band tiles in that order."""
    _alibi_order_case(name, kw, sign, shape, D)


@pytest.mark.parametrize("name,kw,sign", [a for a in ALIBI_ORDER if a[0].startswith("causal")],
                         ids=[a[0] for a in ALIBI_ORDER if a[0].startswith("causal")])
def test_alibi_softmax_tile_order_paired_causal(name, kw, sign):
    """The same on causal rows of the paired core's 4-wavefront workgroups (B2 H16 S4096 D64)."""
    _alibi_order_case(name, kw, sign, PAIRED_CAUSAL, 64)


def _rising_case(name, kw, shape, D):
    B, H, S = shape
    _say(f"[parity] rising scores {name} {shape} D{D}")
    g = torch.Generator("cpu").manual_seed(S + len(name) + D)
    u = torch.randn(D, generator=g)
    u = u / u.norm()
    ramp = torch.arange(S, dtype=torch.float32) * 0.5
    k = (ramp[:, None] * u + 0.3 * torch.randn(B, H, S, D, generator=g)).to(torch.bfloat16)
    q = (4.0 * (D / 64) ** 0.5 * u + 0.3 * torch.randn(B, H, S, D, generator=g)).to(torch.bfloat16)
    v = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16)
    kw = dict(kw)
    if kw.get("head_scale") == "per-head":
        kw["head_scale"] = [0.5 + 0.1 * h for h in range(H)]
    o = attention(q.to(DEV), k.to(DEV), v.to(DEV), **kw)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(o).all()), f"{name}: non-finite output"
    oc = o.float().cpu()
    heads = [(0, 0), (B - 1, H - 1), (B // 2, H // 2)]
    for b, h in heads:
        kwh = dict(kw)
        if "head_scale" in kwh:
            kwh["head_scale"] = [kw["head_scale"][h]]
        r = oracle.attention_ref(q[b:b + 1, h:h + 1], k[b:b + 1, h:h + 1], v[b:b + 1, h:h + 1], **kwh)
        res = gate.north_star_gate(r[0, 0], oc[b, h])
        assert res.ok, f"{name} b={b} h={h}: {res.status} {res.stats}"


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("shape", [(1, 2, 512), (4, 16, 2048)], ids=["B1H2S512", "B4H16S2048"])
@pytest.mark.parametrize("name,kw", RISING, ids=[r[0] for r in RISING])
def test_softmax_rising_scores(name, kw, shape, D):
    """Scores that rise along the keys: q ~ 4 sqrt(D/64) u, k_j ~ (j / 2) u (u a unit vector)
    plus noise, so a row's max climbs ~23 log2-units per 64-key tile at either head dim.  The
    paired core first computes a tile's softmax weights against the running reference max and,
    when a partial row sum over the tile exceeds 2^16, recomputes them against the new max; these
    inputs take that path on almost every tile.  The one-block core does the same per 32-key step
    at head dim 64; at head dim 128 it takes the exact row max of every step, so here they drive
    its per-step rescale of O and l."""
    _rising_case(name, kw, shape, D)


@pytest.mark.parametrize("name,kw", [r for r in RISING if r[0] in ("causal", "softcap50", "headscale")],
                         ids=["causal", "softcap50", "headscale"])
def test_softmax_rising_scores_paired_causal(name, kw):
    """The same on causal rows of the paired core's 4-wavefront workgroups (B2 H16 S4096 D64)."""
    _rising_case(name, kw, PAIRED_CAUSAL, 64)


@pytest.mark.parametrize("cap", [30.0, 54.0])
@pytest.mark.parametrize("shape,D,kw", [((4, 16, 1024), 64, dict(causal=True)), ((1, 2, 512), 64, dict(causal=True, window=300)),
                                        ((1, 2, 512), 128, dict(causal=True))],
                         ids=["B4H16S1024_d64_causal", "B1H2S512_d64_window", "B1H2S512_d128_causal"])
def test_softcap_fixed_reference_saturated(cap, shape, D, kw):
    """Softcap softmax with a cap up to 54 takes its weights against the fixed reference
    cap log2 e - 48 on the one-block core (these shapes run it).  Keys of the first half are
    -50 u and queries 50 u (u a unit vector), so those scores sit at -cap: rows of the first
    half see only weights at the bottom of the range, 2^(48 - 2 cap log2 e), which must stay
    normal; keys of the second half are +50 u, scores at +cap, weights at the top, 2^48."""
    B, H, S = shape
    _say(f"[parity] softcap fixed reference cap={cap} {shape} D{D} {kw}")
    g = torch.Generator("cpu").manual_seed(int(cap) + S + D)
    u = torch.randn(D, generator=g)
    u = u / u.norm()
    sign = torch.where(torch.arange(S) < S // 2, -1.0, 1.0)
    k = (50.0 * sign[:, None] * u + 0.1 * torch.randn(B, H, S, D, generator=g)).to(torch.bfloat16)
    q = (50.0 * u + 0.1 * torch.randn(B, H, S, D, generator=g)).to(torch.bfloat16)
    v = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16)
    o = attention(q.to(DEV), k.to(DEV), v.to(DEV), softcap=cap, **kw)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(o).all())
    oc = o.float().cpu()
    for b, h in [(0, 0), (B - 1, H - 1)]:
        r = oracle.attention_ref(q[b:b + 1, h:h + 1], k[b:b + 1, h:h + 1], v[b:b + 1, h:h + 1], softcap=cap, **kw)
        res = gate.north_star_gate(r[0, 0], oc[b, h])
        assert res.ok, f"cap={cap} b={b} h={h}: {res.status} {res.stats}"


def test_strided_layout_and_out_param():
    """[B, S, H, D] storage viewed as [B, H, S, D] (non-contiguous) and a caller-provided out."""
    _say("[parity] strided layout")
    g = torch.Generator("cpu").manual_seed(5)
    base = [torch.randn(2, 700, 3, 64, generator=g).to(torch.bfloat16) for _ in range(3)]
    q, k, v = (t.to(DEV).transpose(1, 2) for t in base)  # strides (S*H*D, D, H*D, 1)
    out = torch.empty(2, 700, 3, 64, dtype=torch.bfloat16, device=DEV).transpose(1, 2)
    o = attention(q, k, v, causal=True, window=200, out=out)
    assert o.data_ptr() == out.data_ptr()
    torch.cuda.synchronize()
    r = oracle.attention_ref(q.cpu(), k.cpu(), v.cpu(), causal=True, window=200)
    res = gate.north_star_gate(r, o.float().cpu())
    assert res.ok, res.stats


def test_closed_form_row0_and_constant_v():
    """Causal row 0 sees only key 0 (o[0] = v[0]); constant V gives constant O for softmax."""
    _say("[parity] closed forms")
    g = torch.Generator("cpu").manual_seed(9)
    q, k, v = (torch.randn(1, 2, 333, 64, generator=g).to(torch.bfloat16).to(DEV) for _ in range(3))
    o = attention(q, k, v, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(o[:, :, 0], v[:, :, 0])
    vc = torch.full_like(v, 0.75)
    o2 = attention(q, k, vc, causal=False, window=50)
    torch.cuda.synchronize()
    assert (o2.float() - 0.75).abs().max().item() < 4e-3


def test_launch_on_current_stream():
    """The launch is queued on torch's current stream (the reference's behaviour)."""
    _say("[parity] stream")
    g = torch.Generator("cpu").manual_seed(11)
    q, k, v = (torch.randn(1, 2, 512, 64, generator=g).to(torch.bfloat16).to(DEV) for _ in range(3))
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        o = OPS["bias_sliding_window"](q, k, v)
    s.synchronize()
    r = oracle.variant_ref("bias_sliding_window", q.cpu(), k.cpu(), v.cpu())
    res = gate.north_star_gate(r, o.float().cpu())
    assert res.ok, res.stats


def test_deterministic():
    """Two calls give bit-identical outputs (no atomics, fixed reduction order)."""
    g = torch.Generator("cpu").manual_seed(12)
    q, k, v = (torch.randn(2, 4, 1024, 64, generator=g).to(torch.bfloat16).to(DEV) for _ in range(3))
    a = OPS["bias_prefix_lm"](q, k, v)
    b = OPS["bias_prefix_lm"](q, k, v)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_errors_raise_not_abort():
    """Bad inputs raise Python exceptions (reference error behaviour: exceptions, shape_gen.py:97-110)."""
    x = torch.randn(1, 2, 64, 96, device=DEV).to(torch.bfloat16)
    with pytest.raises(ValueError):
        OPS["bias_local"](x, x, x)
    y = torch.randn(1, 2, 64, 64, device=DEV)
    with pytest.raises(TypeError):
        OPS["bias_local"](y, y, y)
    z = torch.randn(1, 2, 64, 64, device=DEV).to(torch.bfloat16)
    with pytest.raises(ValueError):
        attention(z, z, z, dilation=0)
    with pytest.raises(ValueError):
        OPS["temp_perhead"](z, z, z, temperature=[1.0, -1.0])


def test_cached_launch_path_follows_new_data():
    """Repeated calls with one signature reuse the validated arguments: outputs must
    follow new tensors and in-place updates of a device per-head vector."""
    _say("[parity] cached launch path")
    g = torch.Generator("cpu").manual_seed(13)
    q, k, v, q2 = (torch.randn(1, 2, 300, 64, generator=g).to(torch.bfloat16) for _ in range(4))
    qd, kd, vd, q2d = (t.to(DEV) for t in (q, k, v, q2))
    t = torch.tensor([0.5, 2.0], device=DEV)
    for qq, qqd, scale_mult in ((q, qd, 1.0), (q2, q2d, 1.0), (q2, q2d, 3.0)):
        if scale_mult != 1.0:
            t.mul_(scale_mult)  # same storage, new values
        o = attention(qqd, kd, vd, causal=True, window=77, head_scale=t)
        torch.cuda.synchronize()
        r = oracle.attention_ref(qq, k, v, causal=True, window=77, head_scale=t.cpu())
        res = gate.north_star_gate(r, o.float().cpu())
        assert res.ok, res.stats


GQA_CASES = [
    # (name, H, H_kv, S, D, generic kwargs)
    ("causal_g2", 8, 4, 640, 64, dict(causal=True)),
    ("window_g4", 8, 2, 700, 64, dict(causal=True, window=100)),
    ("mqa_alibi", 8, 1, 513, 64, dict(causal=True, alibi_slopes=[0.5 ** (h + 1) for h in range(8)])),
    ("sigmoid_full_g2", 4, 2, 384, 128, dict(norm="sigmoid", causal=False, bias=-2.0)),
    ("relu_block_g4", 4, 1, 300, 64, dict(norm="relu", causal=True, block=64, post_scale=0.05)),
    ("softcap_prefix_g2", 4, 2, 333, 128, dict(causal=True, prefix=70, softcap=20.0)),
]


@pytest.mark.parametrize("name,H,Hkv,S,D,kw", GQA_CASES, ids=[c[0] for c in GQA_CASES])
def test_grouped_query_kv(name, H, Hkv, S, D, kw):
    """K/V with fewer heads than Q (GQA / MQA): bit-identical to the same call with each
    K/V head repeated for its query heads, and within the gate of the oracle."""
    _say(f"[parity] gqa {name}")
    g = torch.Generator("cpu").manual_seed(H * 1000 + Hkv * 10 + S)
    q = torch.randn(2, H, S, D, generator=g).to(torch.bfloat16)
    k, v = (torch.randn(2, Hkv, S, D, generator=g).to(torch.bfloat16) for _ in range(2))
    o = attention(q.to(DEV), k.to(DEV), v.to(DEV), **kw)
    rep = H // Hkv
    o_rep = attention(q.to(DEV), k.repeat_interleave(rep, 1).to(DEV), v.repeat_interleave(rep, 1).to(DEV), **kw)
    torch.cuda.synchronize()
    assert torch.equal(o, o_rep), name
    r = oracle.attention_ref(q, k, v, **kw)
    res = gate.north_star_gate(r, o.float().cpu(), scale_aware=kw.get("norm", "softmax") != "softmax")
    assert res.ok, f"{name}: {res.status} {res.stats}"
