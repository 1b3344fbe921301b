"""SiluAndMul (reference nanovllm/layers/activation.py:6-11) on ``nvx_silu_mul``."""
import torch
from torch import nn

from .. import _C


def silu_and_mul(gate_up):
    N, two_i = gate_up.shape
    inter = two_i // 2
    out = torch.empty(N, inter, dtype=gate_up.dtype, device=gate_up.device)
    _C.require_cuda(gate_up)
    _C.check(_C.lib().nvx_silu_mul(_C.ptr(gate_up), gate_up.stride(0), _C.ptr(out), N, inter,
                                   _C.stream_of(gate_up)))
    return out


class SiluAndMul(nn.Module):

    def forward(self, x):
        return silu_and_mul(x)
