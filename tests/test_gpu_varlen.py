"""Packed variable-length batches on the GPU (attention_varlen / chia_attn_fwd with
cu_seqlens, and its backward): each sequence against the oracle on its own slice,
bit-identity with the fixed-length launch when every sequence has the same
length, the [T, H] lse, empty sequences, and gradients."""
import pytest
import torch

from chia_proj_amd import attention, attention_varlen, gate
from chia_proj_amd.attention import _op_forward, _op_forward_varlen
from oracle.generic import attention_ref
from oracle.grad import attention_grad_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(msg):
    print(msg, flush=True)


def _packed(lens, H, Hkv, D, seed):
    g = torch.Generator("cpu").manual_seed(seed)
    T = sum(lens)
    q = torch.randn(T, H, D, generator=g).to(torch.bfloat16)
    k, v = (torch.randn(T, Hkv, D, generator=g).to(torch.bfloat16) for _ in range(2))
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0).tolist()), dtype=torch.int32)
    return q, k, v, cu


def _seq(t, cu, b):
    """Sequence b of a packed [T, H, D] tensor as [1, H, S_b, D]."""
    return t[int(cu[b]):int(cu[b + 1])].transpose(0, 1).unsqueeze(0)


CASES = [
    # name, lengths, H, Hkv, D, attention() keyword arguments
    ("causal_ragged", [1, 63, 64, 65, 700, 0, 129], 4, 4, 64, dict(causal=True)),
    ("window_dilation", [300, 1000, 5, 257], 2, 2, 64, dict(causal=True, window=100, dilation=3)),
    ("block_prefix_d128", [400, 130, 513], 2, 2, 128, dict(causal=True, block=64, prefix=40)),
    ("local_alibi_softcap_gqa", [333, 777, 2], 4, 2, 64,
     dict(causal=False, window=50, alibi_slopes=[0.1, 0.2, 0.05, 0.3], softcap=15.0)),
    ("sigmoid_headscale", [600, 100, 1], 2, 1, 64, dict(norm="sigmoid", causal=False, bias=-6.0,
                                                     head_scale=[0.5, 2.0])),
    ("relu_block", [256, 500], 2, 2, 128, dict(norm="relu", causal=False, block=128, post_scale=0.01)),
]


@pytest.mark.parametrize("name,lens,H,Hkv,D,kw", CASES, ids=[c[0] for c in CASES])
def test_each_sequence_matches_the_oracle(name, lens, H, Hkv, D, kw):
    _say(f"[varlen] {name}")
    q, k, v, cu = _packed(lens, H, Hkv, D, seed=len(name))
    o = attention_varlen(q.to(DEV), k.to(DEV), v.to(DEV), cu.to(DEV), **kw).cpu()
    for b, L in enumerate(lens):
        if L == 0:
            continue
        ref = attention_ref(_seq(q, cu, b), _seq(k, cu, b), _seq(v, cu, b), **kw)
        got = _seq(o, cu, b).float()
        for h in range(H):
            # sigmoid / ReLU outputs are unnormalised (magnitude grows with the visible
            # keys): the scale-aware gate, as for the variants' unnormalised configurations
            res = gate.north_star_gate(ref[0, h], got[0, h], scale_aware=kw.get("norm", "softmax") != "softmax")
            assert res.ok, (name, b, h, res.status, res.stats)


@pytest.mark.parametrize("kw", [dict(causal=True), dict(causal=True, window=128, dilation=2),
                                dict(norm="sigmoid", causal=False, bias=-5.0)])
def test_equal_lengths_are_bit_identical_to_fixed_length(kw):
    """Same geometry, same per-workgroup work: the packed launch writes exactly
    the fixed-length launch's output (and lse)."""
    _say(f"[varlen] equal lengths {kw}")
    B, S, H = 3, 777, 4
    q, k, v, cu = _packed([S] * B, H, H, 64, seed=5)
    qd, kd, vd, cud = (t.to(DEV) for t in (q, k, v, cu))
    as4 = lambda t: t.view(B, S, t.shape[1], t.shape[2]).transpose(1, 2)  # noqa: E731  [B, H, S, D] views
    o_packed = attention_varlen(qd, kd, vd, cud, **kw)
    o_fixed = attention(as4(qd), as4(kd), as4(vd), **kw)
    assert torch.equal(as4(o_packed), o_fixed)
    if kw.get("norm", "softmax") == "softmax":
        params = dict(norm="softmax", causal=True, window=0, dilation=1, block=0, prefix=0, scale=None,
                      head_scale=None, alibi_slopes=None, softcap=0.0, bias=0.0, post_scale=1.0)
        params.update(kw)
        _, lse_p = _op_forward_varlen(qd, kd, vd, cud, None, params)
        _, lse_f = _op_forward(as4(qd), as4(kd), as4(vd), params)
        assert torch.equal(lse_p.view(B, S, H).transpose(1, 2), lse_f)


def test_dispatch_order_does_not_change_the_result():
    """attention_varlen dispatches the longest sequences first (seq_order); the
    natural order (NULL) writes the same bits: each workgroup's work is the same."""
    _say("[varlen] dispatch order")
    from chia_proj_amd import _lib
    from chia_proj_amd.attention import _prepare_varlen

    q, k, v, cu = _packed([5, 900, 64, 300, 1200], 2, 2, 64, seed=3)
    qd, kd, vd, cud = (t.to(DEV) for t in (q, k, v, cu))
    params = dict(norm="softmax", causal=True, window=0, dilation=1, block=0, prefix=0, scale=None,
                  head_scale=None, alibi_slopes=None, softcap=0.0, bias=0.0, post_scale=1.0)
    o_sorted = attention_varlen(qd, kd, vd, cud)
    a, keep, _, o_nat = _prepare_varlen(qd, kd, vd, cud, None, None, **params)
    a.seq_order = None
    _lib.fwd(a, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(o_sorted, o_nat)


def test_empty_batch_and_max_seqlen():
    _say("[varlen] empty")
    q = torch.empty(0, 2, 64, dtype=torch.bfloat16, device=DEV)
    assert attention_varlen(q, q, q, torch.tensor([0, 0, 0])).shape == (0, 2, 64)
    q, k, v, cu = _packed([10, 0, 30], 2, 2, 64, seed=1)
    a = attention_varlen(q.to(DEV), k.to(DEV), v.to(DEV), cu)
    b = attention_varlen(q.to(DEV), k.to(DEV), v.to(DEV), cu, max_seqlen=200)  # a larger grid, same result
    assert torch.equal(a, b)
    with pytest.raises(ValueError):
        attention_varlen(q.to(DEV), k.to(DEV), v.to(DEV), cu, max_seqlen=20)


@pytest.mark.parametrize("name,lens,H,Hkv,D,kw", [
    ("causal_gqa", [200, 1, 450, 0, 64], 4, 2, 64, dict(causal=True, window=150)),
    ("sigmoid_d128", [300, 129], 2, 2, 128, dict(norm="sigmoid", causal=True, bias=-3.0)),
    ("softcap_block", [513, 77], 2, 1, 64, dict(causal=True, block=100, softcap=10.0)),
], ids=["causal_gqa", "sigmoid_d128", "softcap_block"])
def test_backward_each_sequence(name, lens, H, Hkv, D, kw):
    _say(f"[varlen] backward {name}")
    q, k, v, cu = _packed(lens, H, Hkv, D, seed=7 + len(name))
    do = torch.randn(q.shape, generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)
    qg, kg, vg = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    attention_varlen(qg, kg, vg, cu.to(DEV), **kw).backward(do.to(DEV))
    grads = [t.grad.cpu() for t in (qg, kg, vg)]
    for b, L in enumerate(lens):
        if L == 0:
            continue
        refs = attention_grad_ref(_seq(q, cu, b), _seq(k, cu, b), _seq(v, cu, b), _seq(do, cu, b), **kw)
        floor = 1e-3 * max(r.abs().max().item() for r in refs)
        for label, g, r in zip(("dq", "dk", "dv"), grads, refs):
            got = _seq(g, cu, b).float()
            m = max(r.abs().max().item(), floor, 1e-30)
            err = (got - r).abs()
            assert err.max().item() <= 1e-2 * m and err.mean().item() <= 1e-3 * m, (name, b, label)


def test_backward_equal_lengths_bit_identical():
    _say("[varlen] backward equal lengths")
    B, S, H = 2, 400, 2
    q, k, v, cu = _packed([S] * B, H, H, 64, seed=11)
    do = torch.randn(q.shape, generator=torch.Generator().manual_seed(12)).to(torch.bfloat16).to(DEV)
    as4 = lambda t: t.view(B, S, t.shape[1], t.shape[2]).transpose(1, 2)  # noqa: E731
    g1 = [t.to(DEV).requires_grad_(True) for t in (q, k, v)]
    attention_varlen(*g1, cu.to(DEV), causal=True, window=90).backward(do)
    g2 = [t.to(DEV).requires_grad_(True) for t in (q, k, v)]
    attention(*(as4(t) for t in g2), causal=True, window=90).backward(as4(do))
    for a, b in zip(g1, g2):
        assert torch.equal(a.grad, b.grad)
