"""Empty operands are valid calls that launch nothing and leave the outputs
alone: M = 0 or N = 0 for the matmul family (the reference's linalg ops are
defined on empty shapes), zero rows for the row reductions and zero query
rows for attention."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def test_empty_matmul_family(hx, dev):
    a0 = torch.empty((0, 256), dtype=torch.int8, device=dev)
    b = torch.randint(-127, 128, (256, 256), dtype=torch.int8, device=dev)
    assert hx.gemm_i8(a0, b).shape == (0, 256)
    bz = torch.empty((0, 256), dtype=torch.int8, device=dev)
    assert hx.gemm_i8(torch.ones((8, 256), dtype=torch.int8, device=dev), bz, b_layout="nk").shape == (8, 0)
    x0 = torch.empty((0, 256), dtype=torch.float16, device=dev)
    w = torch.randn((256, 128), dtype=torch.float16, device=dev)
    assert hx.matmul(x0, w).shape == (0, 128)
    s = torch.ones(128, dtype=torch.float16, device=dev)
    assert hx.gemv_w8a16(x0, torch.ones((256, 128), dtype=torch.int8, device=dev), s).shape == (0, 128)
    rw = hx.ResidentWeight(torch.ones((256, 128), dtype=torch.int8, device=dev), s)
    try:
        assert hx.matmul_resident(x0, rw).shape == (0, 128)
    finally:
        rw.release()


def test_empty_rows_and_attention(hx, dev):
    x0 = torch.empty((0, 4096), dtype=torch.float16, device=dev)
    assert hx.softmax(x0).shape == (0, 4096)
    assert hx.rms_norm(x0, torch.ones(4096, dtype=torch.float16, device=dev)).shape == (0, 4096)
    assert hx.layer_norm(x0).shape == (0, 4096)
    q0 = torch.empty((1, 2, 0, 64), dtype=torch.float16, device=dev)
    k = torch.randn((1, 2, 32, 64), dtype=torch.float16, device=dev)
    assert hx.attention(q0, k, k).shape == (1, 2, 0, 64)


def test_attention_without_keys_writes_zeros(hx, dev):
    """Nk = 0: every query has an empty softmax; the kernel writes 0 rather
    than 0/0 (the reference divides acc by l, which stays at its initial
    value for an empty loop; a zero row is the defined result here)."""
    q = torch.randn((1, 1, 40, 64), dtype=torch.float16, device=dev)
    k0 = torch.empty((1, 1, 0, 64), dtype=torch.float16, device=dev)
    out = torch.full_like(q, 7.0)
    hx.attention(q, k0, k0, out=out)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out).item() == 0
