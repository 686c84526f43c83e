"""CPU tests of the unmerged-LoRA helpers (reference comfy_feather/lora.py:4-35):
patch parsing, the separate pass and the factor form used by the fused epilogue."""

from types import SimpleNamespace

import pytest
import torch

from lora_util import make_patches


@pytest.fixture(scope="module")
def lora(pkg):
    from featherops_amd.comfy_feather import lora

    return lora


def test_apply_matches_formula(lora):
    g = torch.Generator().manual_seed(0)
    x = torch.randn(7, 64, generator=g, dtype=torch.float64)
    wf, expect = make_patches(48, 64, [4, 8], g, dtype=torch.float64)
    y0 = torch.randn(7, 48, generator=g, dtype=torch.float64)
    want = y0.clone()
    for down, up, s in expect:  # the reference's own formula, term by term
        want += (x @ down.T) @ up.T * s
    got = lora.apply_lora_patches(x, y0.clone(), wf)
    assert torch.allclose(got, want, rtol=1e-12, atol=1e-12)


def test_alpha_none_means_no_rank_scaling(lora):
    g = torch.Generator().manual_seed(1)
    x = torch.randn(3, 32, generator=g, dtype=torch.float64)
    wf, expect = make_patches(16, 32, [8], g, dtype=torch.float64, alpha=False)
    (down, up, s), = expect
    assert s == pytest.approx(0.8 * 1.25)
    got = lora.apply_lora_patches(x, torch.zeros(3, 16, dtype=torch.float64), wf)
    assert torch.allclose(got, (x @ down.T) @ up.T * s)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_factors_compose_to_the_same_term(lora, dtype):
    """T . U^T over the concatenated, 32-padded rank equals the sum of the
    patches' terms (up to the x-dtype rounding of T)."""
    g = torch.Generator().manual_seed(2)
    x = torch.randn(9, 64, generator=g).to(dtype)
    wf, expect = make_patches(40, 64, [4, 8, 16], g, dtype=dtype)
    t, u = lora.lora_factors(x, wf)
    assert t.shape == (9, 32) and u.shape == (40, 32) and t.dtype == dtype and u.dtype == dtype
    assert t.is_contiguous() and u.is_contiguous()
    assert not t[:, 28:].any() and not u[:, 28:].any()  # zero padding past rank 28
    want = sum((x.double() @ d.double().T) @ up.double().T * s for d, up, s in expect)
    got = t.double() @ u.double().T
    tol = 2**-7 if dtype == torch.bfloat16 else 2**-10
    assert (got - want).abs().max().item() <= tol * want.abs().max().item()


def test_factors_none_without_patches_or_for_fp32(lora):
    g = torch.Generator().manual_seed(3)
    x = torch.randn(4, 32, generator=g)
    wf, _ = make_patches(16, 32, [8], g)
    assert lora.lora_factors(x, wf) is None  # fp32 activations keep the separate pass
    assert lora.lora_factors(x.half(), []) is None
    assert lora.lora_factors(x.half(), [SimpleNamespace(patches={}, key="w")]) is None


@pytest.mark.parametrize("bad", [
    SimpleNamespace(key="w"),                                              # no patches attribute
    SimpleNamespace(patches={"w": [(1.0, SimpleNamespace(), 1.0)]}, key="w"),  # adapter without weights
])
def test_non_basic_patches_raise(lora, bad):
    x = torch.zeros(2, 16, dtype=torch.float16)
    with pytest.raises(NotImplementedError, match="basic LoRA"):
        lora.apply_lora_patches(x, torch.zeros(2, 8, dtype=torch.float16), [bad])
    with pytest.raises(NotImplementedError, match="basic LoRA"):
        lora.lora_factors(x, [bad])


def test_factor_cache_reuse_and_invalidation(lora):
    """The stacked factors are reused while the patches are the same, unmodified
    tensors with the same strengths, and rebuilt when any of that changes."""
    g = torch.Generator().manual_seed(4)
    x = torch.randn(5, 64, generator=g).to(torch.bfloat16)
    wf, _ = make_patches(40, 64, [8, 16], g, dtype=torch.bfloat16)
    cache = {}
    t0, u0 = lora.lora_factors(x, wf, cache)
    entry = cache["entry"]
    t1, u1 = lora.lora_factors(x, wf, cache)
    assert cache["entry"] is entry and u1 is u0 and torch.equal(t1, t0)
    assert torch.equal(t0, lora.lora_factors(x, wf)[0])  # same values as without a cache
    patch = wf[0].patches["w"][0]
    patch[1].weights[0].mul_(2.0)  # up of the first patch changed in place
    _, u2 = lora.lora_factors(x, wf, cache)
    assert cache["entry"] is not entry and torch.equal(u2[:, :8], u0[:, :8] * 2)
    entry = cache["entry"]
    wf[0].patches["w"][0] = (0.5,) + patch[1:]  # new strength
    t3, _ = lora.lora_factors(x, wf, cache)
    assert cache["entry"] is not entry
    assert torch.equal(t3, lora.lora_factors(x, wf)[0])
