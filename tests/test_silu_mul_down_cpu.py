"""silu_mul_down (the MLP tail helper) returns what vLLM's RowParallelLinear.forward returns, so a
model patch that swaps `x, _ = self.down_proj(self.act_fn(gate_up))` for it unpacks the same way.

Run on the CPU through the op's registered fake (FakeTensorMode): only the helper's wrapping is
checked here, not the kernel (tests/test_gpu_silu_linear.py runs it on the GPU)."""
import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

from vllm_sly_radiance_amd import radiance_fused_norm as FN
from vllm_sly_radiance_amd import radiance_mxfp4  # noqa: F401  (registers the radiance ops)

N, K = 64, 512


def down_layer(bias=False, skip_bias_add=False, return_bias=None):
    layer = torch.nn.Module()
    layer.weight = torch.empty((N, K // 2), dtype=torch.uint8)
    layer.weight_scale = torch.empty((N, K // 32), dtype=torch.uint8)
    layer.radiance_wref = torch.empty((N, K, 0), dtype=torch.uint8)
    layer.bias = torch.zeros(N, dtype=torch.bfloat16) if bias else None
    layer.skip_bias_add = skip_bias_add
    if return_bias is not None:
        layer.return_bias = return_bias
    return layer


class MLP(torch.nn.Module):
    """The model's MLP forward with the tail swapped for the helper, unpacking as vLLM's does."""

    def __init__(self, down):
        super().__init__()
        self.down = down

    def forward(self, gate_up):
        x, _ = FN.silu_mul_down(self.down, gate_up)
        return x


@pytest.mark.parametrize("M", [1, 2, 3])
def test_mlp_unpacks_every_row(M):
    with FakeTensorMode():
        down = down_layer()
        x = MLP(down)(torch.empty((M, 2 * K), dtype=torch.bfloat16))
        assert tuple(x.shape) == (M, N)          # not row 0 of an [M, N] output
        x3 = MLP(down)(torch.empty((2, M, 2 * K), dtype=torch.bfloat16))
        assert tuple(x3.shape) == (2, M, N)


def test_bias_follows_skip_bias_add():
    with FakeTensorMode():
        gu = torch.empty((2, 2 * K), dtype=torch.bfloat16)
        y, b = FN.silu_mul_down(down_layer(bias=True), gu)
        assert b is None and tuple(y.shape) == (2, N)
        down = down_layer(bias=True, skip_bias_add=True)
        y, b = FN.silu_mul_down(down, gu)
        assert b is down.bias and tuple(y.shape) == (2, N)
        y = FN.silu_mul_down(down_layer(return_bias=False), gu)
        assert isinstance(y, torch.Tensor) and tuple(y.shape) == (2, N)
