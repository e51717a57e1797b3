"""CPU tests of the Python boundary: the variant registry, parameter mapping,
validation, and the no-fallback rule (no GPU calls are made here)."""
import importlib
import inspect

import pytest
import torch

import oracle
from chia_proj_amd import OPS, OP_NAMES, _lib, attention, core_kwargs
from chia_proj_amd.variants import _spec

REFERENCE_OPS = ["sigmoid_attn", "relu_attn", "temp_perhead", "bias_alibi", "bias_dilated", "bias_local",
                 "bias_block_diagonal", "bias_prefix_lm", "softcap_gemma2", "bias_sliding_window"]


def test_registry_has_the_ten_reference_ops():
    # op names of extra_bench.py:51-62 / the *_BEST.py module names
    assert list(OPS) == REFERENCE_OPS == list(OP_NAMES)
    for op in REFERENCE_OPS:
        mod = importlib.import_module(f"chia_proj_amd.variants.{op}")
        assert mod.launch_kernel is OPS[op]
        params = list(inspect.signature(mod.launch_kernel).parameters)
        assert params[:3] == ["q", "k", "v"]


REFERENCE_MASK = {
    # the constants baked into extra_bench.py:56-61 (plus the causal default, :41)
    "sigmoid_attn": lambda i, j: j <= i,
    "relu_attn": lambda i, j: j <= i,
    "temp_perhead": lambda i, j: j <= i,
    "bias_alibi": lambda i, j: j <= i,
    "softcap_gemma2": lambda i, j: j <= i,
    "bias_dilated": lambda i, j: (j <= i) & (((i - j) % 4) == 0),
    "bias_local": lambda i, j: (i - j).abs() < 256,
    "bias_block_diagonal": lambda i, j: ((i // 512) == (j // 512)) & (j <= i),
    "bias_prefix_lm": lambda i, j: (j <= i) | (j < 256),
    "bias_sliding_window": lambda i, j: (j <= i) & ((i - j) < 256),
}


@pytest.mark.parametrize("op", REFERENCE_OPS)
def test_default_parameters_reproduce_reference_constants(op):
    kw = core_kwargs(op, 32)
    mask_kw = {k: kw[k] for k in ("causal", "window", "dilation", "block", "prefix") if k in kw}
    S = 1100
    i, j = torch.arange(S).view(-1, 1), torch.arange(S).view(1, -1)
    assert torch.equal(oracle.visible_mask(S, **mask_kw), REFERENCE_MASK[op](i, j))
    if op == "temp_perhead":  # TEMP = 0.5 + arange(H)/H in bf16 (extra_bench.py:35)
        ref = (0.5 + torch.arange(32, dtype=torch.bfloat16) / 32).float()
        assert torch.equal(torch.as_tensor(kw["head_scale"]), ref)
    if op == "bias_alibi":  # SLOPE = h + 1 (extra_bench.py:36)
        assert torch.equal(torch.as_tensor(kw["alibi_slopes"]), torch.arange(1, 33, dtype=torch.float32))
    if op == "softcap_gemma2":
        assert kw["softcap"] == 30.0
    if op in ("sigmoid_attn", "relu_attn"):
        assert kw["norm"] == op.split("_")[0]
        assert kw.get("post_scale", 1.0) == 1.0 and kw.get("bias", 0.0) == 0.0


def test_baseline_parameter_forms():
    kw = core_kwargs("temp_perhead", 4, temperature=[0.5, 1.0, 2.0, 4.0], mode="div")
    assert torch.allclose(torch.as_tensor(kw["head_scale"]), torch.tensor([2.0, 1.0, 0.5, 0.25]))
    kw = core_kwargs("bias_alibi", 4, slopes="standard")
    assert torch.allclose(torch.as_tensor(kw["alibi_slopes"]), torch.tensor([2.0 ** (-2 * (h + 1)) for h in range(4)]))
    with pytest.raises(ValueError):
        core_kwargs("temp_perhead", 4, mode="pow")
    with pytest.raises(KeyError):
        core_kwargs("flash", 4)


def test_cpu_tensors_are_rejected_not_computed():
    x = torch.zeros(1, 2, 64, 64, dtype=torch.bfloat16)
    for op in REFERENCE_OPS:
        with pytest.raises(ValueError, match="GPU"):
            OPS[op](x, x, x)


@pytest.mark.parametrize("bad,exc", [
    (lambda: attention(torch.zeros(2, 64, 64), None, None), TypeError),
    (lambda: attention(torch.zeros(1, 2, 64, 64), torch.zeros(1, 2, 64, 64), torch.zeros(1, 2, 64, 64)), TypeError),
    (lambda: attention(*(torch.zeros(2, 64, 64, dtype=torch.bfloat16),) * 3), ValueError),
    (lambda: attention(*(torch.zeros(1, 2, 64, 64, dtype=torch.bfloat16),) * 3, norm="tanh"), ValueError),
    # K/V heads must divide the query heads, and K and V must agree
    (lambda: attention(torch.zeros(1, 6, 64, 64, dtype=torch.bfloat16), *(torch.zeros(1, 4, 64, 64, dtype=torch.bfloat16),) * 2),
     ValueError),
    (lambda: attention(torch.zeros(1, 4, 64, 64, dtype=torch.bfloat16), torch.zeros(1, 2, 64, 64, dtype=torch.bfloat16),
                       torch.zeros(1, 1, 64, 64, dtype=torch.bfloat16)), ValueError),
])
def test_validation_errors(bad, exc):
    with pytest.raises(exc):
        bad()


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libchia_attn.so")
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="not built"):
        _lib.lib()


def test_product_does_not_import_oracle():
    import pathlib

    pkg = pathlib.Path(_lib.__file__).parent
    for path in pkg.rglob("*.py"):
        text = path.read_text()
        assert "import oracle" not in text and "from oracle" not in text, path
