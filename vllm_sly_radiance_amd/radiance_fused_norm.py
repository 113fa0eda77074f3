"""Fused norm / activation + per-token fp8 quant in front of the W4A8 MXFP4 GEMMs (gfx950).

Mirrors sly/mxfp4/radiance_fused_norm.py: the same three custom ops, their fakes, the same gates and
call-site helpers, and the same switches. Each op ends in the per-token e4m3 quantizer
radiance::mxfp4_linear runs internally, so its (q, scale) pair goes straight to
radiance::mxfp4_linear_pq (apply_weights' tuple branch) instead of a bf16 tensor that the op
re-quantizes:

  add_rms_quant   Gemma RMSNorm with residual (decoder input / post-attention layernorm): fp32 add,
                  x * rsqrt(mean(x^2) + eps) * (w + 1) -> bf16 -> e4m3, plus the bf16 residual out.
  silu_mul_quant  MLP act_fn: silu(gate) * up -> e4m3 for down_proj.
  gdn_norm_quant  GatedDeltaNet output projection: per-head RMSNormGated (norm before gate, silu
                  gate) -> e4m3 for out_proj; z may be a column slice of the fused projection.

The HIP library does the work (w4a8_add_rms_quant / w4a8_silu_mul_quant / w4a8_gdn_norm_quant);
there is no torch fallback. Each op's result equals "the producer's bf16 output, then the plain
quantizer" bit for bit (the quantizer divides by the scale, as _traced_quant does).

Not carried over from the reference: the fragment-tiled q layout (the MI355X GEMM reads row-major
activations through LDS at the same rate either way), the fp8 hi/lo activation split and the online
Hadamard rotation (both belong to checkpoint variants outside this path).

Switches (read once at import, as the reference does): RADIANCE_FUSED_NORM_QUANT=1 arms the fusions
(default off), RADIANCE_FUSED_NORM_QUANT_ADD_RMS / _SILU / _GDN (default 1 each) pick them.
"""
from __future__ import annotations

import os

import torch

from . import _native


def _flag(name: str, default: str) -> bool:
    return os.environ.get(name, default) == "1"


ENABLED = _flag("RADIANCE_FUSED_NORM_QUANT", "0")
ADD_RMS = ENABLED and _flag("RADIANCE_FUSED_NORM_QUANT_ADD_RMS", "1")
SILU = ENABLED and _flag("RADIANCE_FUSED_NORM_QUANT_SILU", "1")
GDN = ENABLED and _flag("RADIANCE_FUSED_NORM_QUANT_GDN", "1")

# Launcher limits (sly/mxfp4/radiance_fused_norm.py:48-52): add_rms K <= 10240, silu N <= 18432,
# gdn N <= 10240 with 128-wide heads; all 8-aligned.
ADD_RMS_MAX_K = 10240
SILU_MAX_N = 18432
GDN_MAX_N = 10240
GDN_HEAD = 128


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _check_bf16(name: str, *ts: torch.Tensor) -> None:
    for t in ts:
        if t.dtype != torch.bfloat16:
            raise RuntimeError(f"radiance::{name}: expected bfloat16, got {t.dtype}")


def _qs(M: int, K: int, device):
    return (torch.empty((M, K), device=device, dtype=torch.float8_e4m3fn),
            torch.empty((M,), device=device, dtype=torch.float32))


# ---- custom ops -------------------------------------------------------------------------------
@torch.library.custom_op("radiance::add_rms_quant", mutates_args=())
def add_rms_quant_op(y: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                     eps: float) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """y, residual: [M, K] bf16; weight: [K] bf16 (Gemma convention, the kernel adds the 1).
    Returns (q [M, K] e4m3, scale [M] f32, residual_out [M, K] bf16)
    (sly/mxfp4/radiance_fused_norm.py:132-152)."""
    _check_bf16("add_rms_quant", y, residual, weight)
    M, K = y.shape
    q, s = _qs(M, K, y.device)
    r = torch.empty((M, K), device=y.device, dtype=torch.bfloat16)
    if M:
        y, residual, weight = y.contiguous(), residual.contiguous(), weight.contiguous()
        _native.add_rms_quant(y.data_ptr(), residual.data_ptr(), weight.data_ptr(), q.data_ptr(),
                              s.data_ptr(), r.data_ptr(), M, K, float(eps), _stream())
    return q, s, r


@add_rms_quant_op.register_fake
def _(y, residual, weight, eps):
    M, K = y.shape
    return (torch.empty((M, K), device=y.device, dtype=torch.float8_e4m3fn),
            torch.empty((M,), device=y.device, dtype=torch.float32),
            torch.empty((M, K), device=y.device, dtype=torch.bfloat16))


@torch.library.custom_op("radiance::silu_mul_quant", mutates_args=())
def silu_mul_quant_op(gate_up: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """gate_up: [M, 2N] bf16 -> (q [M, N] e4m3 of silu(gate) * up, scale [M] f32)
    (sly/mxfp4/radiance_fused_norm.py:163-180)."""
    _check_bf16("silu_mul_quant", gate_up)
    M, N2 = gate_up.shape
    N = N2 // 2
    q, s = _qs(M, N, gate_up.device)
    if M:
        gate_up = gate_up.contiguous()
        _native.silu_mul_quant(gate_up.data_ptr(), q.data_ptr(), s.data_ptr(), M, N, _stream())
    return q, s


@silu_mul_quant_op.register_fake
def _(gate_up):
    M, N2 = gate_up.shape
    return (torch.empty((M, N2 // 2), device=gate_up.device, dtype=torch.float8_e4m3fn),
            torch.empty((M,), device=gate_up.device, dtype=torch.float32))


@torch.library.custom_op("radiance::gdn_norm_quant", mutates_args=())
def gdn_norm_quant_op(x: torch.Tensor, z: torch.Tensor, weight: torch.Tensor,
                      eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """x: [M, N] bf16 (N = heads * 128); z: [M, N] bf16, any row stride as long as each row is a
    contiguous run; weight: [128] bf16. Returns (q [M, N] e4m3, scale [M] f32)
    (sly/mxfp4/radiance_fused_norm.py:189-213)."""
    _check_bf16("gdn_norm_quant", x, z, weight)
    M, N = x.shape
    q, s = _qs(M, N, x.device)
    if M:
        x, weight = x.contiguous(), weight.contiguous()
        if M > 1 and (z.stride(1) != 1 or z.stride(0) < N or z.stride(0) % 8):
            z = z.contiguous()
        elif M == 1 and z.stride(1) != 1:
            z = z.contiguous()
        zs = int(z.stride(0)) if M > 1 else N
        if z.data_ptr() % 16:
            z = z.contiguous()
            zs = N
        _native.gdn_norm_quant(x.data_ptr(), z.data_ptr(), zs, weight.data_ptr(), q.data_ptr(),
                               s.data_ptr(), M, N, float(eps), _stream())
    return q, s


@gdn_norm_quant_op.register_fake
def _(x, z, weight, eps):
    M, N = x.shape
    return (torch.empty((M, N), device=x.device, dtype=torch.float8_e4m3fn),
            torch.empty((M,), device=x.device, dtype=torch.float32))


# ---- gates (traced; plain attribute reads only) -------------------------------------------------
# The reference tests isinstance against vLLM's GemmaRMSNorm / RMSNormGated / SiluAndMul; vLLM is
# not a dependency here, so the gates compare class names, which is the same test when vLLM is
# present (sly/mxfp4/radiance_fused_norm.py:226-299).
def _is(obj, name: str) -> bool:
    return any(c.__name__ == name for c in type(obj).__mro__)


def mx_ok(lin) -> bool:
    """A radiance W4A8 linear whose apply_weights takes the (q, scale) tuple branch."""
    return (getattr(lin, "radiance_w4a8_ok", False)
            and getattr(lin, "radiance_wref", None) is not None
            and not getattr(lin, "_rad_ar_overlap", False)
            and getattr(lin, "tp_size", 1) == 1)


def _gemma_ok(norm) -> bool:
    w = getattr(norm, "weight", None)
    return (norm is not None and _is(norm, "GemmaRMSNorm") and w is not None
            and w.dtype == torch.bfloat16 and w.shape[0] % 8 == 0
            and w.shape[0] <= ADD_RMS_MAX_K)


def input_ok(layer) -> bool:
    """Decoder input_layernorm (residual != None) -> the attention's projections."""
    if getattr(layer, "use_attn_reduce_scatter_for_moe", True):
        return False
    if not _gemma_ok(getattr(layer, "input_layernorm", None)):
        return False
    kind = getattr(layer, "layer_type", None)
    if kind == "linear_attention":
        a = layer.linear_attn
        return (getattr(a, "tp_size", 0) == 1 and mx_ok(getattr(a, "in_proj_qkvz", None))
                and mx_ok(getattr(a, "in_proj_ba", None)))
    if kind == "full_attention":
        return mx_ok(getattr(layer.self_attn, "qkv_proj", None))
    return False


def post_ok(layer) -> bool:
    """Decoder post_attention_layernorm -> dense MLP gate_up_proj."""
    if getattr(layer, "use_attn_reduce_scatter_for_moe", True):
        return False
    if not _gemma_ok(getattr(layer, "post_attention_layernorm", None)):
        return False
    mlp = getattr(layer, "mlp", None)
    return getattr(mlp, "expert_gate", 1) is None and mx_ok(getattr(mlp, "gate_up_proj", None))


def mlp_ok(mlp) -> bool:
    """MLP act_fn (SiluAndMul) -> down_proj."""
    d = getattr(mlp, "down_proj", None)
    if not (_is(getattr(mlp, "act_fn", None), "SiluAndMul") and mx_ok(d)):
        return False
    n = int(getattr(d, "radiance_wref").shape[1])        # down_proj's K = the act width N
    return n % 8 == 0 and n <= SILU_MAX_N


def gdn_ok(attn) -> bool:
    """GatedDeltaNet _output_projection -> out_proj."""
    n = getattr(attn, "norm", None)
    if not (n is not None and _is(n, "RMSNormGated") and mx_ok(getattr(attn, "out_proj", None))):
        return False
    return (getattr(attn, "tp_size", 0) == 1 and getattr(attn, "head_v_dim", 0) == GDN_HEAD
            and getattr(n, "group_size", None) is None and getattr(n, "norm_before_gate", False)
            and getattr(n, "activation", None) in ("silu", "swish")
            and n.weight.dtype == torch.bfloat16 and n.weight.shape[0] == GDN_HEAD
            and getattr(attn, "value_dim", GDN_MAX_N + 1) <= GDN_MAX_N)


# ---- call sites (traced) ----------------------------------------------------------------------
def add_rms_quant(norm, hidden_states: torch.Tensor, residual: torch.Tensor):
    """GemmaRMSNorm(hidden_states, residual) + quant -> ((q, scale), residual_out)."""
    q, s, r = torch.ops.radiance.add_rms_quant(hidden_states, residual, norm.weight,
                                               norm.variance_epsilon)
    return (q, s), r


def silu_mul_quant(gate_up: torch.Tensor):
    q, s = torch.ops.radiance.silu_mul_quant(gate_up)
    return (q, s)


def gdn_norm_quant(attn, core_attn_out: torch.Tensor, z: torch.Tensor):
    """_output_projection's norm(core_attn_out, z) + flatten + quant -> (q, scale)."""
    M = core_attn_out.shape[0]
    q, s = torch.ops.radiance.gdn_norm_quant(core_attn_out.reshape(M, -1), z.reshape(M, -1),
                                             attn.norm.weight, attn.norm.eps)
    return (q, s)
