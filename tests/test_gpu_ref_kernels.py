"""GPU parity of the drop-in ``qabs_cuda_kernels`` functions against the
restated reference kernels: fp32 scores bit-exact (same accumulation order,
no FMA contraction), attention within 1e-2 / 2e-2 of fp64."""

import numpy as np
import pytest
import torch

from kv_cache_amd import qabs_cuda_kernels as Q
from oracle import ref_semantics as R

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.bfloat16, torch.float16, torch.float32]


def f32(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("dim_count", [1, 8, 32, 128, 500])
def test_partial_scores(dtype, dim_count):
    g = torch.Generator().manual_seed(dim_count)
    q = torch.randn((2, 4, 128), generator=g).to(dtype)
    q[0, 0, 5] = q[0, 0, 9] = 3.0            # a |q| tie: lower dim first
    k = torch.randn((2, 4, 700, 128), generator=g).to(dtype)
    out = Q.partial_scores(q.to(DEV), k.to(DEV), dim_count)
    want = R.partial_scores(f32(q), f32(k), dim_count)
    assert out.dtype == torch.float32 and out.shape == (2, 4, 700)
    assert np.array_equal(out.cpu().numpy(), want)


def test_partial_scores_strided_key():
    g = torch.Generator().manual_seed(1)
    q = torch.randn((1, 2, 64), generator=g).to(torch.bfloat16)
    kdm = torch.randn((1, 2, 64, 300), generator=g).to(torch.bfloat16)
    k = kdm.transpose(2, 3)                    # token-major view of dim-major storage
    out = Q.partial_scores(q.to(DEV), kdm.to(DEV).transpose(2, 3), 16)
    assert np.array_equal(out.cpu().numpy(), R.partial_scores(f32(q), f32(k), 16))


@pytest.mark.parametrize("dtype", DTYPES)
def test_partial_scores_dim_major(dtype):
    g = torch.Generator().manual_seed(2)
    q = torch.randn((3, 2, 128), generator=g).to(dtype)
    kdm = torch.randn((3, 2, 128, 1000), generator=g).to(dtype)
    idx = torch.topk(q.float().abs(), 24, dim=-1).indices
    out = Q.partial_scores_dim_major(q.to(DEV), kdm.to(DEV), idx.to(DEV))
    assert np.array_equal(out.cpu().numpy(), R.partial_scores_dim_major(f32(q), f32(kdm), idx.numpy()))
    # growing-capacity cache view as the reference keeps it (EV:2029-2042)
    cap = torch.zeros((3, 2, 128, 1500), dtype=dtype)
    cap[..., :1000] = kdm
    out2 = Q.partial_scores_dim_major(q.to(DEV), cap.to(DEV)[..., :1000], idx.to(DEV))
    assert torch.equal(out2.cpu(), out.cpu())


@pytest.mark.parametrize("dtype", DTYPES)
def test_candidate_full_scores(dtype):
    g = torch.Generator().manual_seed(3)
    q = torch.randn((2, 3, 128), generator=g).to(dtype)
    k = torch.randn((2, 3, 400, 128), generator=g).to(dtype)
    cur = torch.rand((2, 3, 400), generator=g) < 0.1
    prev = torch.rand((2, 3, 400), generator=g) < 0.1
    fin = torch.rand((2, 3, 400), generator=g) < 0.05
    for p, f, sink, recent in [(None, None, 0, 0), (prev, None, 4, 0), (prev, fin, 10, 10), (None, fin, 0, 7)]:
        out = Q.candidate_full_scores(q.to(DEV), k.to(DEV), cur.to(DEV), None if p is None else p.to(DEV),
                                      None if f is None else f.to(DEV), sink, recent, 0.088)
        want = R.candidate_full_scores(f32(q), f32(k), cur.numpy(), None if p is None else p.numpy(),
                                       None if f is None else f.numpy(), sink, recent, 0.088)
        assert np.array_equal(out.cpu().numpy(), want)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [1, 37, 256, 2051])
def test_final_attention(dtype, n):
    g = torch.Generator().manual_seed(n)
    b, h, t = 2, 4, 3000
    q = torch.randn((b, h, 128), generator=g).to(dtype)
    k = torch.randn((b, h, t, 128), generator=g).to(dtype)
    v = torch.randn((b, h, t, 128), generator=g).to(dtype)
    idx = torch.randint(0, t, (b, h, n), generator=g)
    valid = torch.rand((b, h, n), generator=g) < 0.9
    idx[0, 0, 0] = t + 5          # out of range: ignored
    idx[0, 1, 0] = -3
    valid[1, 2] = False           # nothing valid: zeros
    out = Q.final_attention(q.to(DEV), k.to(DEV), v.to(DEV), idx.to(DEV), valid.to(DEV), 128 ** -0.5)
    assert out.shape == (b, 1, h, 128) and out.dtype == dtype
    want = R.final_attention(f32(q), f32(k), f32(v), idx.numpy(), valid.numpy(), 128 ** -0.5)
    assert np.allclose(f32(out), want, rtol=1e-2, atol=2e-2)
    assert torch.count_nonzero(out[1, 0, 2].float()) == 0


def test_reference_error_messages():
    q = torch.zeros((1, 2, 8), device=DEV)
    with pytest.raises(RuntimeError, match="query/key shape mismatch"):
        Q.partial_scores(q, torch.zeros((1, 2, 4, 16), device=DEV), 2)
    with pytest.raises(RuntimeError, match="dim_indices must be int64"):
        Q.partial_scores_dim_major(q, torch.zeros((1, 2, 8, 4), device=DEV), torch.zeros((1, 2, 2), dtype=torch.int32, device=DEV))
    with pytest.raises(RuntimeError, match="current_candidate must be bool"):
        Q.candidate_full_scores(q, torch.zeros((1, 2, 4, 8), device=DEV), torch.zeros((1, 2, 4), device=DEV),
                                None, None, 0, 0, 1.0)
    with pytest.raises(RuntimeError, match="indices must be int64"):
        Q.final_attention(q, torch.zeros((1, 2, 4, 8), device=DEV), torch.zeros((1, 2, 4, 8), device=DEV),
                          torch.zeros((1, 2, 3), dtype=torch.int32, device=DEV),
                          torch.ones((1, 2, 3), dtype=torch.bool, device=DEV), 1.0)
