"""RMSNorm (reference nanovllm/layers/layernorm.py:16-40) on the fused HIP kernel
``nvx_rmsnorm``: plain and add+RMSNorm, same numerics (fp32 statistics, bf16
rounding of the normalised value, then the weight)."""
import torch
from torch import nn

from .. import _C


def rms_norm(x, weight, eps, residual=None):
    """x [N, H] bf16 (unit stride in H); returns out, or (out, residual_out)."""
    N, H = x.shape
    out = torch.empty(N, H, dtype=x.dtype, device=x.device)
    res_out = None
    if residual is not None:
        residual = residual.contiguous()
        res_out = torch.empty_like(out)
    _C.require_cuda(x, weight, residual)
    _C.check(_C.lib().nvx_rmsnorm(_C.ptr(x), x.stride(0), _C.ptr(residual), _C.ptr(res_out),
                                  _C.ptr(weight), _C.ptr(out), N, H, float(eps), _C.stream_of(x)))
    return out if residual is None else (out, res_out)


class RMSNorm(nn.Module):

    def __init__(self, hidden_size: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(hidden_size))

    def forward(self, x, residual=None):
        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        if x2.stride(-1) != 1:
            x2 = x2.contiguous()
        if residual is None:
            return rms_norm(x2, self.weight, self.eps).view(shape)
        out, res = rms_norm(x2, self.weight, self.eps, residual.reshape(-1, shape[-1]))
        return out.view(shape), res.view(shape)
