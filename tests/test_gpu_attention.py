"""GPU parity for the fused attention forward (hx_attention) against the CPU
oracle and, at the reference test's configuration, against torch's
scaled_dot_product_attention with the reference's bound
(test/python/triton/test_flash_attention.py: Z = H = 1, N_CTX = 1024,
D_HEAD = 64, scale 0.5, torch.rand inputs, relative Frobenius error < 5e-3)."""
import numpy as np
import pytest
import torch

from conftest import bf16_from_f32, rng, to_dev, to_np

import oracle

pytestmark = pytest.mark.gpu


def rel_err(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / np.linalg.norm(want))


def test_attention_reference_config(hx, dev):
    torch.manual_seed(0)
    q, k, v = (torch.rand(1, 1, 1024, 64) for _ in range(3))
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, v, scale=0.5)
    out = hx.attention(q.half().to(dev), k.half().to(dev), v.half().to(dev), scale=0.5)
    got = out.float().cpu().numpy()
    assert rel_err(got, ref.numpy()) < 5e-3
    want = oracle.attention(q.half().numpy(), k.half().numpy(), v.half().numpy(), 0.5)
    assert np.abs(got - want.astype(np.float32)).max() < 2e-3


@pytest.mark.parametrize("shape", [(2, 3, 333, 333, 64), (1, 2, 200, 517, 128), (1, 1, 64, 64, 64),
                                   (2, 2, 130, 1, 64), (1, 4, 1000, 1000, 128),
                                   (1, 1, 200, 700, 64), (1, 1, 700, 200, 128), (1, 2, 100, 1500, 64)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("causal", [False, True])
def test_attention_vs_oracle(hx, dev, shape, causal):
    """Causal masks key j for query i when j > i, for any Nq and Nk (query i
    always sees key 0).  The (1, 1, ...) and (1, 2, 100, 1500) shapes leave
    fewer than 128 (head, query block) workgroups, so their key range is
    split and merged; with Nq != Nk under the mask the split ranges past a
    row's diagonal carry only masked keys."""
    Z, H, Nq, Nk, D = shape
    r = rng(Nq * 7 + Nk + D + int(causal))
    q = r.normal(0, 1, (Z, H, Nq, D)).astype(np.float16)
    k = r.normal(0, 1, (Z, H, Nk, D)).astype(np.float16)
    v = r.normal(0, 1, (Z, H, Nk, D)).astype(np.float16)
    scale = D ** -0.5
    got = to_np(hx.attention(to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), scale=scale, causal=causal))
    want = oracle.attention(q, k, v, scale, causal=causal)
    assert np.abs(got.astype(np.float32) - want.astype(np.float32)).max() < 1e-2
    assert rel_err(got, want) < 3e-3


def test_attention_bf16(hx, dev):
    r = rng(77)
    q, k, v = (bf16_from_f32(r.normal(0, 1, (1, 2, 256, 64)).astype(np.float32)) for _ in range(3))
    bf = lambda a: to_dev(a.view(np.int16), dev).view(torch.bfloat16)  # noqa: E731
    out = hx.attention(bf(q), bf(k), bf(v), scale=0.125)
    got = to_np(out)
    want = oracle.attention(q, k, v, 0.125, bf16=True)
    g = oracle.bf16_bits_to_f32(got.view(np.uint16))
    w = oracle.bf16_bits_to_f32(want.view(np.uint16))
    assert np.abs(g - w).max() < 3e-2 and rel_err(g, w) < 1e-2


def test_attention_strided_heads_and_determinism(hx, dev):
    """[Z, N, H, D] storage viewed as [Z, H, N, D] (the usual projection
    layout): strided N and H dims, innermost D contiguous."""
    Z, N, H, D = 2, 300, 4, 64
    r = rng(5)
    x = [r.normal(0, 1, (Z, N, H, D)).astype(np.float16) for _ in range(3)]
    td = [to_dev(a, dev).permute(0, 2, 1, 3) for a in x]
    got = to_np(hx.attention(*td, scale=0.125))
    again = to_np(hx.attention(*td, scale=0.125))
    assert np.array_equal(got.view(np.uint16), again.view(np.uint16))
    want = oracle.attention(*(np.ascontiguousarray(a.transpose(0, 2, 1, 3)) for a in x), 0.125)
    assert np.abs(got.astype(np.float32) - want.astype(np.float32)).max() < 1e-2


@pytest.mark.parametrize("causal", [False, True])
def test_attention_split_matches_single_pass(hx, dev, causal):
    """One head alone occupies 8 workgroups, so its key range is split and
    the partials merged; the same head repeated 128 times fills the chip and
    runs in a single pass.  Both agree with each other and with the oracle."""
    r = rng(91 + int(causal))
    q, k, v = (r.normal(0, 1, (1, 1, 1024, 64)).astype(np.float16) for _ in range(3))
    split = to_np(hx.attention(to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), scale=0.125, causal=causal))
    rep = [to_dev(a, dev).repeat(1, 128, 1, 1) for a in (q, k, v)]
    single = to_np(hx.attention(*rep, scale=0.125, causal=causal))
    assert all(np.array_equal(single[:, 0].view(np.uint16), single[:, h].view(np.uint16)) for h in range(128))
    want = oracle.attention(q, k, v, 0.125, causal=causal).astype(np.float32)
    s32, p32 = split.astype(np.float32), single[:, :1].astype(np.float32)
    assert np.abs(s32 - p32).max() < 2e-3
    assert np.abs(s32 - want).max() < 1e-2 and rel_err(s32, want) < 3e-3
    assert np.abs(p32 - want).max() < 1e-2 and rel_err(p32, want) < 3e-3


def test_attention_rejects_bad_head_dim(hx, dev):
    q = torch.zeros((1, 1, 64, 96), dtype=torch.float16, device=dev)
    with pytest.raises(hx.HXError, match="head-dim"):
        hx.attention(q, q, q)
