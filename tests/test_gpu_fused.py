"""Fused model layers (HIP) vs plain PyTorch fp32 restatements of the reference
layers (layernorm.py:16-40, rotary_embedding.py:6-14, activation.py:8-11)."""
import pytest
import torch

from nanovllm.layers.activation import silu_and_mul
from nanovllm.layers.layernorm import rms_norm
from nanovllm.layers.rotary_embedding import RotaryEmbedding
from nanovllm import _C


def ref_rms(x, w, eps, residual=None):
    x = x.float()
    if residual is not None:
        x = x + residual.float()
        residual = x.to(torch.bfloat16)
    var = x.pow(2).mean(-1, keepdim=True)
    y = (x * torch.rsqrt(var + eps)).to(torch.bfloat16)
    y = (y.float() * w.float()).to(torch.bfloat16)
    return y if residual is None else (y, residual)


def ulps(a, b):
    """Distance in bf16 ulps (both bf16)."""
    ai = a.view(torch.int16).int()
    bi = b.view(torch.int16).int()
    ai = torch.where(ai < 0, -(ai & 0x7fff), ai)
    bi = torch.where(bi < 0, -(bi & 0x7fff), bi)
    return (ai - bi).abs()


@pytest.mark.gpu
# Hidden sizes of the Qwen3 family and two others, 257 rows each.
@pytest.mark.parametrize("H", [4096, 3072, 2048, 1024, 1536, 128])
def test_rmsnorm_plain_and_add(dev, H):
    g = torch.Generator().manual_seed(H)
    x = torch.randn(257, H, generator=g).to(torch.bfloat16)
    r = torch.randn(257, H, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16)
    # the normalised value is rounded to bf16 before the weight multiply (as in the
    # reference), so a 1-ulp difference in rsqrt can surface as 2 ulps
    y = rms_norm(x.to(dev), w.to(dev), 1e-6).cpu()
    d = ulps(y, ref_rms(x, w, 1e-6))
    assert d.max() <= 2 and d.float().mean() < 0.05
    y2, r2 = rms_norm(x.to(dev), w.to(dev), 1e-6, r.to(dev))
    ey, er = ref_rms(x, w, 1e-6, r)
    assert torch.equal(r2.cpu(), er)
    d = ulps(y2.cpu(), ey)
    assert d.max() <= 2 and d.float().mean() < 0.05


@pytest.mark.gpu
# Head layouts of Qwen3-8B (32/8) and Qwen3-0.6B (16/8) and two others, with token
# counts that leave a partial last workgroup.
@pytest.mark.parametrize("N,Hq,Hkv", [(300, 8, 2), (301, 32, 8), (77, 16, 8), (50, 12, 4)])
def test_qk_norm_rope(dev, N, Hq, Hkv):
    g = torch.Generator().manual_seed(N)
    D = 128
    qkv = torch.randn(N, (Hq + 2 * Hkv) * D, generator=g).to(torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    pos = torch.randint(0, 5000, (N,), generator=g)
    rope = RotaryEmbedding(D, D, 8192, 1000000.0)
    q_ref = ref_rms(qkv[:, :Hq * D].reshape(N, Hq, D), qw, 1e-6)
    k_ref = ref_rms(qkv[:, Hq * D:(Hq + Hkv) * D].reshape(N, Hkv, D), kw, 1e-6)
    q_ref, k_ref = rope(pos, q_ref, k_ref)
    # device copies are bound to names: a temporary freed after its pointer is taken
    # could be handed to the next allocation before the kernel runs
    qd, kd = qkv.to(dev), torch.empty(N, Hkv, D, dtype=torch.bfloat16, device=dev)
    q = torch.empty(N, Hq, D, dtype=torch.bfloat16, device=dev)
    cs, qwd, kwd, posd = rope.cos_sin_cache.to(dev), qw.to(dev), kw.to(dev), pos.to(dev)
    _C.check(_C.lib().nvx_qk_norm_rope(_C.ptr(qd), qd.stride(0), Hq, Hkv, D, _C.ptr(qwd),
                                       _C.ptr(kwd), _C.ptr(posd), _C.ptr(cs), N,
                                       _C.ptr(q), _C.ptr(kd), 1e-6, _C.stream_of(qd)))
    torch.cuda.synchronize()
    # RoPE mixes two rounded values (x1*cos - x2*sin), so outputs near zero can
    # differ by many ulps while the absolute error stays at bf16 resolution
    for a, b in ((q.cpu().float(), q_ref.float()), (kd.cpu().float(), k_ref.float())):
        err = (a - b).abs()
        assert float(err.max()) < 3e-2, float(err.max())
        assert float((err / (b.abs() + 1e-2)).mean()) < 2e-3


@pytest.mark.gpu
def test_silu_mul(dev):
    g = torch.Generator().manual_seed(1)
    x = (torch.randn(129, 2 * 3072, generator=g) * 3).to(torch.bfloat16)
    out = silu_and_mul(x.to(dev)).cpu()
    gte, up = x.float().chunk(2, -1)
    ref = (torch.nn.functional.silu(gte) * up).to(torch.bfloat16)
    d = ulps(out, ref)
    assert d.max() <= 1 and d.float().mean() < 0.05
