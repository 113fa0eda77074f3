"""Fused norm / activation + per-token fp8 quant in front of the W4A8 MXFP4 GEMMs (gfx950).

Interface of sly/mxfp4/radiance_fused_norm.py, kept so that the reference's model patch
(sly/patch_fused_norm_quant.py) drives this module unchanged: the three custom ops with their
fakes, the switch names, the gate names (mx_ok, input_ok, post_ok, mlp_ok, gdn_ok) and the
call-site helper names and signatures. Each op ends in the per-token e4m3 quantizer that
radiance::mxfp4_linear runs internally, so its (q, scale) pair goes straight to
radiance::mxfp4_linear_pq (apply_weights' tuple branch) instead of a bf16 tensor that the op
re-quantizes:

  add_rms_quant   Gemma RMSNorm with residual: fp32 add, x * rsqrt(mean(x^2) + eps) * (w + 1)
                  -> bf16 -> e4m3, plus the bf16 residual out.
  silu_mul_quant  silu(gate) * up -> e4m3.
  gdn_norm_quant  per-head gated RMSNorm (norm before gate, silu gate) -> e4m3; z may be a column
                  slice of a wider projection.

The HIP library does the work (w4a8_add_rms_quant / w4a8_silu_mul_quant / w4a8_gdn_norm_quant);
there is no torch fallback. Each op's result equals "the producer's bf16 output, then the plain
quantizer" bit for bit (the quantizer divides by the scale, as _traced_quant does).

When a fusion is valid is data here, not code: SITES lists each place in a decoder where a
producer can stand in for a bf16 activation (which module produces it, which linears consume it,
what the host module must look like), and one function, site_ok, checks a site against a module.
The gates are thin names over it. Everything they read is a plain attribute, so a tracing compiler
folds each gate to a constant per layer.

At M >= RADIANCE_MXFP4_A_TILED_MIN_M (radiance_mxfp4; default off) the add-RMSNorm and SiLU-mul
producers write q fragment-tiled, in the order the tile GEMM reads (w4a8_gemm_at), and record it in
radiance_mxfp4's TiledHandoff for mxfp4_linear_pq; the gated norm does too when
RADIANCE_MXFP4_TILED_OPROJ=1. The codes and scales are the same bytes in either layout; the choice is
made per call from eager ints inside the opaque op body.

Not carried over: the fp8 hi/lo activation split and the online Hadamard rotation (both belong to
checkpoint variants outside this path).

Switches, read once at import: RADIANCE_FUSED_NORM_QUANT=1 arms the fusions (default off);
RADIANCE_FUSED_NORM_QUANT_ADD_RMS / _SILU / _GDN (default 1 each) then pick them;
RADIANCE_MXFP4_TILED_OPROJ=1 lets the gated norm write the tiled layout (default off, as in the
reference, sly/mxfp4/radiance_fused_norm.py:40-42).
"""
from __future__ import annotations

import os
from dataclasses import dataclass, field

import torch

from . import _native
from . import radiance_mxfp4 as _rmx

_MASTER = "RADIANCE_FUSED_NORM_QUANT"


def _armed(fusion: str) -> bool:
    """A fusion is on when the master switch is "1" and its own switch (default "1") is too."""
    env = os.environ
    return env.get(_MASTER, "0") == "1" and env.get(f"{_MASTER}_{fusion}", "1") == "1"


ENABLED = os.environ.get(_MASTER, "0") == "1"
ADD_RMS, SILU, GDN = (_armed(f) for f in ("ADD_RMS", "SILU", "GDN"))
TILED_OPROJ = os.environ.get("RADIANCE_MXFP4_TILED_OPROJ", "0") == "1"

# Widths the producer kernels accept (the entry points refuse anything else): add-RMSNorm rows up
# to 10240, SiLU-mul outputs up to 18432, gated-norm rows up to 10240 in 128-wide heads; all
# multiples of 8. The same limits as the reference's launchers.
ADD_RMS_MAX_K = 10240
SILU_MAX_N = 18432
GDN_MAX_N = 10240
GDN_HEAD = 128


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _need_bf16(op: str, **tensors: torch.Tensor) -> None:
    bad = {k: t.dtype for k, t in tensors.items() if t.dtype != torch.bfloat16}
    if bad:
        raise RuntimeError(f"radiance::{op}: bfloat16 inputs required, got {bad}")


def _row_runs(t: torch.Tensor, n: int):
    """(t, row stride) such that every row of t is n contiguous elements starting 16-byte aligned,
    one stride apart, which is all the gated-norm kernel needs of z. A column slice of a wider
    bf16 projection qualifies as it is; anything else is copied to a contiguous tensor first."""
    rows = t.shape[0]
    stride = int(t.stride(0)) if rows > 1 else n
    fits = t.stride(1) == 1 and t.data_ptr() % 16 == 0 and stride >= n and stride % 8 == 0
    if not fits:
        t, stride = t.contiguous(), n
    return t, stride


def _tiled(M: int, K: int) -> bool:
    """Write this producer's q fragment-tiled: the consumer GEMM's M asks for it and the row is
    whole 128-byte k-tiles."""
    return _rmx.a_tiled_wanted(M) and K % 128 == 0


def _qs(M: int, K: int, device, tiled: bool = False):
    q = (_rmx.alloc_tiled_q(M, K, device) if tiled
         else torch.empty((M, K), device=device, dtype=torch.float8_e4m3fn))
    return q, torch.empty((M,), device=device, dtype=torch.float32)


def _layout(q: torch.Tensor, M: int, K: int, tiled: bool) -> int:
    """The q_layout argument; a tiled q is recorded for its consumers (queued before any of them
    can run, since they take q from this op's return)."""
    if not tiled:
        return _native.Q_ROWS
    _rmx.a_tiled_register(q, M, K)
    return _native.Q_TILED


# ---- custom ops -------------------------------------------------------------------------------
@torch.library.custom_op("radiance::add_rms_quant", mutates_args=())
def add_rms_quant_op(y: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                     eps: float) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """y, residual: [M, K] bf16; weight: [K] bf16 (Gemma convention, the kernel adds the 1).
    Returns (q [M, K] e4m3, scale [M] f32, residual_out [M, K] bf16)
    (sly/mxfp4/radiance_fused_norm.py:132-152)."""
    _need_bf16("add_rms_quant", y=y, residual=residual, weight=weight)
    M, K = y.shape
    tiled = _tiled(M, K)
    q, s = _qs(M, K, y.device, tiled)
    r = torch.empty((M, K), device=y.device, dtype=torch.bfloat16)
    if M:
        y, residual, weight = y.contiguous(), residual.contiguous(), weight.contiguous()
        _native.add_rms_quant(y.data_ptr(), residual.data_ptr(), weight.data_ptr(), q.data_ptr(),
                              s.data_ptr(), r.data_ptr(), M, K, float(eps), _stream(),
                              _layout(q, M, K, tiled))
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
    _need_bf16("silu_mul_quant", gate_up=gate_up)
    M, N2 = gate_up.shape
    N = N2 // 2
    tiled = _tiled(M, N)
    q, s = _qs(M, N, gate_up.device, tiled)
    if M:
        gate_up = gate_up.contiguous()
        _native.silu_mul_quant(gate_up.data_ptr(), q.data_ptr(), s.data_ptr(), M, N, _stream(),
                               _layout(q, M, N, tiled))
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
    _need_bf16("gdn_norm_quant", x=x, z=z, weight=weight)
    M, N = x.shape
    tiled = TILED_OPROJ and _tiled(M, N)
    q, s = _qs(M, N, x.device, tiled)
    if M:
        # every copy stays referenced until the launch is queued
        x, weight = x.contiguous(), weight.contiguous()
        z, zs = _row_runs(z, N)
        _native.gdn_norm_quant(x.data_ptr(), z.data_ptr(), zs, weight.data_ptr(), q.data_ptr(),
                               s.data_ptr(), M, N, float(eps), _stream(), _layout(q, M, N, tiled))
    return q, s


@gdn_norm_quant_op.register_fake
def _(x, z, weight, eps):
    M, N = x.shape
    return (torch.empty((M, N), device=x.device, dtype=torch.float8_e4m3fn),
            torch.empty((M,), device=x.device, dtype=torch.float32))


# ---- where a fusion is valid ------------------------------------------------------------------
_ABSENT = object()


def _at(obj, path):
    """The attribute at a dotted path ("mlp.gate_up_proj"), or _ABSENT when a link is missing."""
    if path is None:
        return None
    for name in path.split("."):
        obj = getattr(obj, name, _ABSENT)
        if obj is _ABSENT:
            break
    return obj


def _is(obj, name: str) -> bool:
    """Class-name test against the MRO: vLLM is not a dependency here, and with vLLM present a
    GemmaRMSNorm / SiluAndMul / RMSNormGated instance carries exactly that name."""
    return any(c.__name__ == name for c in type(obj).__mro__)


# Predicates on one attribute value; an absent attribute fails all of them but `_unset`.
def _eq(v):
    return lambda x: x is not _ABSENT and x == v


def _le(v):
    return lambda x: x is not _ABSENT and x <= v


def _one_of(*vs):
    return lambda x: x is not _ABSENT and x in vs


def _falsy(x):
    return x is not _ABSENT and not x


def _truthy(x):
    return x is not _ABSENT and bool(x)


def _none(x):
    return x is None


def _unset(x):
    return x is None or x is _ABSENT


def _bf16_vector(multiple_of=1, at_most=None, exactly=None):
    """A bf16 tensor whose leading size fits the producer kernel."""
    def ok(t):
        if not isinstance(t, torch.Tensor) or t.dtype != torch.bfloat16:
            return False
        n = t.shape[0]
        return n % multiple_of == 0 and (at_most is None or n <= at_most) \
            and (exactly is None or n == exactly)
    return ok


def _k_of_descriptor(at_most):
    """The K a radiance linear's (N, K, 0) layout descriptor records: 8-aligned and in range."""
    def ok(ref):
        return isinstance(ref, torch.Tensor) and ref.dim() == 3 \
            and ref.shape[1] % 8 == 0 and ref.shape[1] <= at_most
    return ok


@dataclass(frozen=True)
class Site:
    """One place where a producer's (q, scale) output can stand in for a bf16 activation.

    producer / producer_class: the module (a dotted path from the host module) whose output the
        fused op replaces, and the class it must be.
    consumers: host kind -> the linears that read the activation; every one of them must be a
        radiance W4A8 linear (mx_ok), or the unfused chain stays. `kind_attr` names the host
        attribute that picks the kind; without it the single entry under None applies.
    requires: (path, predicate) pairs the host must satisfy, plus `by_kind` ones per kind.
    """
    producer: str
    producer_class: str
    consumers: dict
    requires: tuple = ()
    by_kind: dict = field(default_factory=dict)
    kind_attr: str | None = None


def _gemma(path):
    return ((f"{path}.weight", _bf16_vector(multiple_of=8, at_most=ADD_RMS_MAX_K)),)


# The reduce-scatter MoE path hands the norm output to a collective, not to the linears.
_NO_REDUCE_SCATTER = (("use_attn_reduce_scatter_for_moe", _falsy),)

SITES = {
    # decoder input norm (with residual) -> the attention block's input projections
    "input": Site(
        producer="input_layernorm", producer_class="GemmaRMSNorm", kind_attr="layer_type",
        consumers={"linear_attention": ("linear_attn.in_proj_qkvz", "linear_attn.in_proj_ba"),
                   "full_attention": ("self_attn.qkv_proj",)},
        requires=_NO_REDUCE_SCATTER + _gemma("input_layernorm"),
        by_kind={"linear_attention": (("linear_attn.tp_size", _eq(1)),)}),
    # post-attention norm -> a dense MLP's fused gate/up projection (a MoE block has an expert
    # gate, which reads the bf16 activation itself)
    "post": Site(
        producer="post_attention_layernorm", producer_class="GemmaRMSNorm",
        consumers={None: ("mlp.gate_up_proj",)},
        requires=_NO_REDUCE_SCATTER + (("mlp.expert_gate", _none),)
        + _gemma("post_attention_layernorm")),
    # MLP activation -> down projection; the activation width is down's K
    "mlp": Site(
        producer="act_fn", producer_class="SiluAndMul", consumers={None: ("down_proj",)},
        requires=(("down_proj.radiance_wref", _k_of_descriptor(SILU_MAX_N)),)),
    # GatedDeltaNet output norm (per 128-wide head, norm before the silu gate) -> out_proj
    "gdn": Site(
        producer="norm", producer_class="RMSNormGated", consumers={None: ("out_proj",)},
        requires=(("tp_size", _eq(1)), ("head_v_dim", _eq(GDN_HEAD)),
                  ("value_dim", _le(GDN_MAX_N)), ("norm.group_size", _unset),
                  ("norm.norm_before_gate", _truthy), ("norm.activation", _one_of("silu", "swish")),
                  ("norm.weight", _bf16_vector(exactly=GDN_HEAD)))),
}


def mx_ok(lin) -> bool:
    """A radiance W4A8 linear whose apply_weights takes the (q, scale) tuple branch: repacked by
    this plugin, not under the all-reduce overlap wrapper, not tensor-parallel."""
    return (_truthy(_at(lin, "radiance_w4a8_ok"))
            and _at(lin, "radiance_wref") not in (None, _ABSENT)
            and not _truthy(_at(lin, "_rad_ar_overlap"))
            and getattr(lin, "tp_size", 1) == 1)


def site_ok(site: Site, host) -> bool:
    """Whether `host` (a decoder layer, MLP or attention module) matches `site`."""
    kind = _at(host, site.kind_attr)
    consumers = site.consumers.get(kind)
    if consumers is None or not _is(_at(host, site.producer), site.producer_class):
        return False
    for path, ok in site.requires + site.by_kind.get(kind, ()):
        if not ok(_at(host, path)):
            return False
    for path in consumers:
        if not mx_ok(_at(host, path)):
            return False
    return True


# ---- gates (names the model patch calls) --------------------------------------------------------
def input_ok(layer) -> bool:
    return site_ok(SITES["input"], layer)


def post_ok(layer) -> bool:
    return site_ok(SITES["post"], layer)


def mlp_ok(mlp) -> bool:
    return site_ok(SITES["mlp"], mlp)


def gdn_ok(attn) -> bool:
    return site_ok(SITES["gdn"], attn)


# ---- call-site helpers (names and signatures the model patch calls) -----------------------------
def add_rms_quant(norm, hidden_states: torch.Tensor, residual: torch.Tensor):
    """Stands in for norm(hidden_states, residual): returns ((q, scale), new residual)."""
    q, scale, new_residual = torch.ops.radiance.add_rms_quant(
        hidden_states, residual, norm.weight, norm.variance_epsilon)
    return (q, scale), new_residual


def silu_mul_quant(gate_up: torch.Tensor):
    """Stands in for act_fn(gate_up): returns (q, scale)."""
    return tuple(torch.ops.radiance.silu_mul_quant(gate_up))


def silu_mul_down(down, gate_up: torch.Tensor):
    """Stands in for down(act_fn(gate_up)) when `down` is a layer this plugin serves: the
    SiLU-and-mul and the down projection in one op (one launch at M <= 2; the same bits as
    down(silu_mul_quant(gate_up))).

    Returns what vLLM's RowParallelLinear.forward returns, so the model's `x, _ = down(...)`
    unpacks it unchanged: (output, output_bias), where the bias is added to output unless the
    layer has skip_bias_add (then output_bias is the bias, else None), or output alone when the
    layer has return_bias = False."""
    lead = gate_up.shape[:-1]
    y = torch.ops.radiance.silu_mul_mxfp4_linear(gate_up.reshape(-1, gate_up.shape[-1]),
                                                 down.weight, down.weight_scale,
                                                 down.radiance_wref)
    bias = getattr(down, "bias", None)
    skip = bool(getattr(down, "skip_bias_add", False))
    if bias is not None and not skip:
        y = y + bias
    y = y.reshape(*lead, y.shape[-1])
    if not getattr(down, "return_bias", True):
        return y
    return y, (bias if skip else None)


def gdn_norm_quant(attn, core_attn_out: torch.Tensor, z: torch.Tensor):
    """Stands in for attn.norm(core_attn_out, z) flattened to one row per token: (q, scale)."""
    tokens = core_attn_out.shape[0]
    return tuple(torch.ops.radiance.gdn_norm_quant(
        core_attn_out.reshape(tokens, -1), z.reshape(tokens, -1), attn.norm.weight, attn.norm.eps))
