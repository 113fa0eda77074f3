"""The fused-producer gates on stand-in decoder modules (CPU, no vLLM).

Each site fuses only when every condition holds: the producer is the right module, every consumer
is a radiance W4A8 linear and the host looks as the kernel needs (sly/mxfp4/radiance_fused_norm.py
:226-288 states the same conditions). The tests build a module tree that passes each gate, then
break one condition at a time and check that the gate declines; a missing attribute declines too,
except where the condition is "unset" (a gated norm without group_size)."""
import copy
import types

import pytest
import torch

from vllm_sly_radiance_amd import radiance_fused_norm as FN


class GemmaRMSNorm(torch.nn.Module):
    def __init__(self, k):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.zeros(k, dtype=torch.bfloat16))
        self.variance_epsilon = 1e-6


class RMSNormGated(torch.nn.Module):
    def __init__(self, head=128):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.ones(head, dtype=torch.bfloat16))
        self.group_size = None
        self.norm_before_gate = True
        self.activation = "silu"
        self.eps = 1e-6


class SiluAndMul(torch.nn.Module):
    pass


class RMSNorm(torch.nn.Module):          # a norm of another kind: never fused
    def __init__(self, k):
        super().__init__()
        self.weight = torch.nn.Parameter(torch.zeros(k, dtype=torch.bfloat16))


def radiance_linear(N, K):
    lin = types.SimpleNamespace()
    lin.radiance_w4a8_ok = True
    lin.radiance_wref = torch.empty((N, K, 0), dtype=torch.uint8)
    lin.tp_size = 1
    return lin


def plain_linear():
    return types.SimpleNamespace(weight=torch.zeros(4, 4))


def decoder(kind):
    layer = types.SimpleNamespace(layer_type=kind, use_attn_reduce_scatter_for_moe=False)
    layer.input_layernorm = GemmaRMSNorm(5120)
    layer.post_attention_layernorm = GemmaRMSNorm(5120)
    if kind == "linear_attention":
        layer.linear_attn = types.SimpleNamespace(
            tp_size=1, in_proj_qkvz=radiance_linear(12288, 5120),
            in_proj_ba=radiance_linear(96, 5120))
    else:
        layer.self_attn = types.SimpleNamespace(qkv_proj=radiance_linear(10240, 5120))
    layer.mlp = types.SimpleNamespace(expert_gate=None, gate_up_proj=radiance_linear(17408, 5120),
                                      act_fn=SiluAndMul(), down_proj=radiance_linear(5120, 8704))
    return layer


def gdn_attn():
    return types.SimpleNamespace(norm=RMSNormGated(), out_proj=radiance_linear(5120, 6144),
                                 tp_size=1, head_v_dim=128, value_dim=6144)


def test_switches_default_off():
    assert FN.ENABLED is False and not (FN.ADD_RMS or FN.SILU or FN.GDN)


@pytest.mark.parametrize("kind", ["linear_attention", "full_attention"])
def test_gates_accept_a_conforming_tree(kind):
    layer = decoder(kind)
    assert FN.input_ok(layer) and FN.post_ok(layer) and FN.mlp_ok(layer.mlp)
    assert FN.gdn_ok(gdn_attn())


def _declines(gate, host, path, value):
    """Whether `gate` declines a copy of `host` with the attribute at `path` set to `value`
    (deleted for _DELETE)."""
    h = copy.deepcopy(host)
    *parents, leaf = path.split(".")
    obj = h
    for p in parents:
        obj = getattr(obj, p)
    if value is _DELETE:
        delattr(obj, leaf)
    else:
        setattr(obj, leaf, value)
    return not gate(h)


_DELETE = object()

INPUT_BREAKS = [
    ("use_attn_reduce_scatter_for_moe", True),
    ("use_attn_reduce_scatter_for_moe", _DELETE),
    ("input_layernorm", RMSNorm(5120)),
    ("input_layernorm.weight", torch.nn.Parameter(torch.zeros(5120, dtype=torch.float32))),
    ("input_layernorm.weight", torch.nn.Parameter(torch.zeros(5124, dtype=torch.bfloat16))),
    ("input_layernorm.weight", torch.nn.Parameter(torch.zeros(10248, dtype=torch.bfloat16))),
    ("layer_type", "mamba"),
    ("layer_type", _DELETE),
]


@pytest.mark.parametrize("kind", ["linear_attention", "full_attention"])
@pytest.mark.parametrize("path,value", INPUT_BREAKS)
def test_input_gate_declines(kind, path, value):
    assert _declines(FN.input_ok, decoder(kind), path, value)


@pytest.mark.parametrize("path,value", [
    ("linear_attn.tp_size", 2),
    ("linear_attn.tp_size", _DELETE),
    ("linear_attn.in_proj_ba", plain_linear()),
    ("linear_attn.in_proj_qkvz.radiance_w4a8_ok", False),
    ("linear_attn.in_proj_qkvz._rad_ar_overlap", True),
    ("linear_attn.in_proj_qkvz.tp_size", 2),
    ("linear_attn.in_proj_ba.radiance_wref", None),
])
def test_input_gate_declines_linear_attention(path, value):
    assert _declines(FN.input_ok, decoder("linear_attention"), path, value)


def test_input_gate_full_attention_consumer():
    assert _declines(FN.input_ok, decoder("full_attention"), "self_attn.qkv_proj", plain_linear())


@pytest.mark.parametrize("path,value", [
    ("use_attn_reduce_scatter_for_moe", True),
    ("post_attention_layernorm", RMSNorm(5120)),
    ("post_attention_layernorm.weight", torch.nn.Parameter(torch.zeros(4, dtype=torch.float16))),
    ("mlp.expert_gate", torch.nn.Linear(4, 1)),
    ("mlp.expert_gate", _DELETE),
    ("mlp.gate_up_proj", plain_linear()),
    ("mlp.gate_up_proj", _DELETE),
])
def test_post_gate_declines(path, value):
    assert _declines(FN.post_ok, decoder("full_attention"), path, value)


@pytest.mark.parametrize("path,value", [
    ("act_fn", torch.nn.GELU()),
    ("down_proj", plain_linear()),
    ("down_proj.radiance_wref", torch.empty((5120, 8708, 0), dtype=torch.uint8)),
    ("down_proj.radiance_wref", torch.empty((5120, 18440, 0), dtype=torch.uint8)),
])
def test_mlp_gate_declines(path, value):
    assert _declines(FN.mlp_ok, decoder("full_attention").mlp, path, value)


def test_mlp_gate_width_limit_is_inclusive():
    mlp = decoder("full_attention").mlp
    mlp.down_proj = radiance_linear(5120, FN.SILU_MAX_N)
    assert FN.mlp_ok(mlp)


@pytest.mark.parametrize("path,value", [
    ("norm", RMSNorm(128)),
    ("out_proj", plain_linear()),
    ("tp_size", 2),
    ("tp_size", _DELETE),
    ("head_v_dim", 64),
    ("head_v_dim", _DELETE),
    ("value_dim", 10368),
    ("value_dim", _DELETE),
    ("norm.group_size", 64),
    ("norm.norm_before_gate", False),
    ("norm.norm_before_gate", _DELETE),
    ("norm.activation", "sigmoid"),
    ("norm.weight", torch.nn.Parameter(torch.ones(64, dtype=torch.bfloat16))),
    ("norm.weight", torch.nn.Parameter(torch.ones(128, dtype=torch.float32))),
])
def test_gdn_gate_declines(path, value):
    assert _declines(FN.gdn_ok, gdn_attn(), path, value)


def test_gdn_gate_accepts_swish_and_absent_group_size():
    attn = gdn_attn()
    attn.norm.activation = "swish"
    del attn.norm.group_size
    assert FN.gdn_ok(attn)
    attn.value_dim = FN.GDN_MAX_N
    assert FN.gdn_ok(attn)


def test_mx_ok_defaults():
    lin = radiance_linear(16, 512)
    del lin.tp_size                       # not tensor-parallel unless it says so
    assert FN.mx_ok(lin)
    assert not FN.mx_ok(None)
    assert not FN.mx_ok(plain_linear())


def test_row_runs_keeps_a_column_slice_and_copies_the_rest():
    wide = torch.zeros((4, 3 * 256), dtype=torch.bfloat16)
    z = wide[:, 256:512]                  # a column slice: rows contiguous, stride 768
    t, stride = FN._row_runs(z, 256)
    assert t.data_ptr() == z.data_ptr() and stride == 768
    zt = torch.zeros((256, 4), dtype=torch.bfloat16).t()   # column-major: copied
    t, stride = FN._row_runs(zt, 256)
    assert t.is_contiguous() and stride == 256
    t, stride = FN._row_runs(wide[:1, 256:512], 256)        # one row: stride is the width
    assert stride == 256
