"""MI355X (gfx950) MXFP4 W4A8 linear path behind the reference's vLLM plugin surface.

Mirrors sly/mxfp4/radiance_mxfp4.py: the same custom ops (radiance::mxfp4_linear,
radiance::mxfp4_linear_pq, :644, :825), the same MxFp4LinearKernel plugin methods
(is_supported / can_implement / process_weights_after_loading / apply_weights, :1016-1217) plus the
quant-method name apply(), and the same refuse-never-silently-wrong rules. The numerics are W4A8:
e2m1 weights with e8m0 per-32 block scales times per-token e4m3 activations, fp32 accumulation, bf16
out. The HIP library does all the device work; there is no torch or CPU fallback on this path, and
a missing library raises.

What changes underneath: on CDNA4 the scaled MFMA applies the e8m0 block scale itself, so the load
step is one repack into "MFMA granules" (w4a8_repack) instead of permute_w + psw_pack_w_ +
psw_fold_ws + make_row_ref. After process_weights_after_loading a layer holds:
  weight          uint8 [Np, Kp/2]   granules (N padded to 16, K to 512; same storage when aligned)
  weight_scale    uint8 [Np, Kp/32]  scale dwords viewed as bytes
  radiance_wref   uint8 (N, K, 0)    zero-size layout descriptor carrying the logical N and K in
                                     its shape (the reference's per-row max exponent has no use
                                     here; keeping the attribute keeps apply_weights branch-free)
"""
from __future__ import annotations

import os
import sys
from collections import OrderedDict

import torch

from . import _native
from . import diagnostics as _diag

ENABLED = os.environ.get("RADIANCE_MXFP4_W4A8", "0") == "1"
# The registered split-K scratch covers every automatic plan up to these M and N (the decode band,
# where the plan may split K across workgroups, ends at M = 64).
SCRATCH_MAX_N = int(os.environ.get("RADIANCE_MXFP4_SCRATCH_MAX_N", "36864"))
SCRATCH_MAX_M = 64
ACTIVATION_QUANT_KEY = "kMxfp4Dynamic"

# Fragment-tiled activations (sly/mxfp4/radiance_mxfp4.py:29-39): the producers of
# radiance_fused_norm write q in the layout the tile GEMM reads as contiguous 1 KiB units
# (w4a8_gemm_at) when M >= this; 0 = off. Below M = 65 the streaming and ring kernels, which read
# row-major activations, are faster than any macro tile, so the threshold must lie above that band.
A_TILED_MIN_M = int(os.environ.get("RADIANCE_MXFP4_A_TILED_MIN_M", "0"))
DECODE_BAND_MAX_M = 64
if A_TILED_MIN_M and A_TILED_MIN_M <= DECODE_BAND_MAX_M:
    raise RuntimeError(f"RADIANCE_MXFP4_A_TILED_MIN_M must exceed {DECODE_BAND_MAX_M} (the decode "
                       f"band reads row-major activations), got {A_TILED_MIN_M}")

STATS = {"fast": 0, "refused": 0, "calls": 0, "calls_pq": 0, "calls_tiled": 0, "calls_silu": 0}
_scratch = [None, None]          # [partials, counters]: torch-owned, alive for the process


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


# --------------------------------------------------------------------------------------------
# Device operations on torch tensors
# --------------------------------------------------------------------------------------------
def quant_per_token(x: torch.Tensor):
    """bf16 [M, K] -> (e4m3fn [M, K], fp32 [M]). Semantics of _traced_quant
    (sly/mxfp4/radiance_mxfp4.py:392-396), computed by the HIP quantizer."""
    if x.dtype != torch.bfloat16 or x.dim() != 2 or x.stride(1) != 1:
        raise RuntimeError(f"[radiance.mxfp4] quant needs a 2-D bf16 tensor with unit column "
                           f"stride, got {tuple(x.shape)} {x.dtype} stride {x.stride()}")
    M, K = x.shape
    q = torch.empty((M, K), dtype=torch.float8_e4m3fn, device=x.device)
    s = torch.empty((M,), dtype=torch.float32, device=x.device)
    _native.quant_per_token(x.data_ptr(), x.stride(0), q.data_ptr(), s.data_ptr(), M, K,
                            _stream())
    return q, s


def repack_weights(weight: torch.Tensor, weight_scale: torch.Tensor):
    """Checkpoint (weight [N, K/2] uint8, weight_scale [N, K/32] uint8) -> granules (wq, sq) as
    uint8 [Np, Kp/2] and [Np, Kp/32]."""
    N, K = weight.shape[0], weight.shape[1] * 2
    if weight.dtype != torch.uint8 or weight_scale.dtype != torch.uint8 \
            or tuple(weight_scale.shape) != (N, K // 32):
        raise RuntimeError(f"[radiance.mxfp4] repack needs weight [N, K/2] and weight_scale "
                           f"[N, K/32] uint8, got {tuple(weight.shape)} {weight.dtype} / "
                           f"{tuple(weight_scale.shape)} {weight_scale.dtype}")
    w = weight.contiguous()
    ws = weight_scale.contiguous()
    wq_bytes, sq_bytes = _native.packed_bytes(N, K)
    Np, Kp = -(-N // 16) * 16, -(-K // 512) * 512
    wq = torch.empty((Np, Kp // 2), dtype=torch.uint8, device=w.device)
    sq = torch.empty((Np, Kp // 32), dtype=torch.uint8, device=w.device)
    assert wq.numel() == wq_bytes and sq.numel() == sq_bytes
    _native.repack(w.data_ptr(), ws.data_ptr(), wq.data_ptr(), sq.data_ptr(), N, K, _stream())
    return wq, sq


# --------------------------------------------------------------------------------------------
# Fragment-tiled handoff, producer -> consumer
# --------------------------------------------------------------------------------------------
def a_tiled_wanted(M: int) -> bool:
    """Should a producer of M tokens write q fragment-tiled (sly/mxfp4/radiance_mxfp4.py:50-51)."""
    return A_TILED_MIN_M > 0 and M >= A_TILED_MIN_M


def alloc_tiled_q(M: int, K: int, device) -> torch.Tensor:
    """An [M, K] e4m3 tensor over storage of whole 16-token blocks (w4a8_tiled_bytes) plus a
    128-byte tail that nothing reads: the tail gives tiled storage a size no row-major [M', K]
    tensor has, which TiledHandoff checks. Rows are a view, so real and fake shapes agree."""
    mp = -(-M // 16) * 16
    buf = torch.empty((mp * K + 128,), dtype=torch.float8_e4m3fn, device=device)
    return buf[:mp * K].view(mp, K)[:M]


class TiledHandoff:
    """Which pre-quantized activations are fragment-tiled. A tensor's bytes do not say how they are
    ordered, and the custom-op boundary carries tensors only, so the producer records the tensor
    it wrote (data pointer -> M, K, storage bytes) and mxfp4_linear_pq looks its input up, as the
    reference does through its data_ptr table (sly/mxfp4/radiance_mxfp4.py:54-80).

    A record stays after a lookup (a gated-norm q feeds two linears), and goes when its address is
    marked again, when a lookup finds another shape or storage size there, or when it is older than
    the last `keep` marks. A lookup needs the same (M, K) and the tiled storage size (whole blocks
    plus the 128-byte tail, which no row-major [M', K] allocation has), so a row-major tensor at a
    recycled address reads as row-major unless it is a view into that same tiled storage; callers
    that quantized row-major themselves pass allow_tiled=False and skip the lookup."""

    def __init__(self, keep: int = 64):
        self.keep = keep
        self._rec: OrderedDict[int, tuple[int, int, int]] = OrderedDict()

    @staticmethod
    def _sig(q: torch.Tensor, M: int, K: int) -> tuple[int, int, int]:
        return (M, K, q.untyped_storage().nbytes() - q.storage_offset() * q.element_size())

    def mark(self, q: torch.Tensor, M: int, K: int) -> None:
        ptr = q.data_ptr()
        self._rec.pop(ptr, None)
        self._rec[ptr] = self._sig(q, M, K)
        while len(self._rec) > self.keep:
            self._rec.popitem(last=False)

    def claim(self, q: torch.Tensor, M: int, K: int) -> bool:
        ptr = q.data_ptr()
        rec = self._rec.get(ptr)
        if rec is None:
            return False
        mp = -(-M // 16) * 16
        if rec != self._sig(q, M, K) or rec[2] != mp * K + 128:
            del self._rec[ptr]
            return False
        return True

    def clear(self) -> None:
        self._rec.clear()


A_TILED = TiledHandoff()


def a_tiled_register(q: torch.Tensor, M: int, K: int) -> None:
    """Record q (written fragment-tiled by a producer) for its consumers
    (sly/mxfp4/radiance_mxfp4.py:66-71)."""
    A_TILED.mark(q, M, K)


def a_tiled_take(q: torch.Tensor, M: int, K: int) -> bool:
    """Is q a recorded fragment-tiled tensor of this shape (sly/mxfp4/radiance_mxfp4.py:74-81)."""
    return A_TILED.claim(q, M, K)


def layout_ref(N: int, K: int, device) -> torch.Tensor:
    """The zero-size (N, K, 0) descriptor stored as layer.radiance_wref."""
    return torch.empty((N, K, 0), dtype=torch.uint8, device=device)


def ensure_scratch(device) -> None:
    """Allocate and register the split-K scratch once per process, at load time (outside graph
    capture), torch-owned, as the reference does (sly/mxfp4/radiance_mxfp4.py:1054-1080). Sized
    by the library from its own plan: what any M <= SCRATCH_MAX_M, N <= SCRATCH_MAX_N may use."""
    if _scratch[0] is not None:
        return
    part_bytes, cnt_bytes = _native.workspace_bytes(SCRATCH_MAX_M, SCRATCH_MAX_N)
    partial = torch.empty(max(part_bytes, 16) // 4, dtype=torch.float32, device=device)
    counters = torch.zeros(max(cnt_bytes, 4) // 4, dtype=torch.int32, device=device)
    _native.set_scratch(partial.data_ptr(), partial.numel() * 4, counters.data_ptr(),
                        counters.numel() * 4)
    _scratch[0], _scratch[1] = partial, counters


def gemm(x_fp8: torch.Tensor, x_scale: torch.Tensor, weight: torch.Tensor,
         weight_scale: torch.Tensor, N: int, K: int, out: torch.Tensor | None = None,
         kernel: int = 0, variant: int = -1, split_k: int = 0) -> torch.Tensor:
    M = x_fp8.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=x_fp8.device)
    _native.gemm(x_fp8.data_ptr(), x_scale.data_ptr(), weight.data_ptr(), weight_scale.data_ptr(),
                 out.data_ptr(), M, N, K, _stream(), kernel, variant, split_k)
    return out


# --------------------------------------------------------------------------------------------
# Custom ops: the whole path is one opaque node (sly/mxfp4/radiance_mxfp4.py:644-652)
# --------------------------------------------------------------------------------------------
@torch.library.custom_op("radiance::mxfp4_linear", mutates_args=())
def mxfp4_linear(x: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor,
                 weight_ref: torch.Tensor) -> torch.Tensor:
    """bf16 x [M, K] -> bf16 [M, N]: per-token e4m3 quant + W4A8 GEMM on the current stream. At
    M <= 2 (M <= 4 where the plan leaves its quantizing waves little work) one launch quantizes
    beside the streaming GEMM, else two launches; the bits are the same either way. N and K come
    from weight_ref's shape (see module docstring)."""
    STATS["calls"] += 1
    _diag.report_stats(STATS)
    N, K = weight_ref.shape[0], weight_ref.shape[1]
    if x.dim() != 2 or x.shape[1] != K:
        raise RuntimeError(f"[radiance.mxfp4] x {tuple(x.shape)} does not match K={K}")
    if x.dtype != torch.bfloat16 or x.stride(1) != 1:
        raise RuntimeError(f"[radiance.mxfp4] x must be bf16 with unit column stride, got "
                           f"{x.dtype} stride {x.stride()}")
    M = x.shape[0]
    x = _diag.sanitize(x)
    out = _diag.new_out(M, N, x.device)
    q = torch.empty((M, K), dtype=torch.float8_e4m3fn, device=x.device)
    s = torch.empty((M,), dtype=torch.float32, device=x.device)
    _native.linear(x.data_ptr(), x.stride(0), q.data_ptr(), s.data_ptr(), weight.data_ptr(),
                   weight_scale.data_ptr(), out.data_ptr(), M, N, K, _stream())
    if _diag.enabled():
        # the one-launch form keeps q in LDS: the check quantizes again (the same bits)
        _diag.after_call(STATS, lambda: quant_per_token(x), None, weight, weight_scale, out, N, K,
                         x=x)
    return _diag.returned(out)


@mxfp4_linear.register_fake
def _(x, weight, weight_scale, weight_ref):
    return torch.empty((x.shape[0], weight_ref.shape[0]), device=x.device, dtype=torch.bfloat16)


@torch.library.custom_op("radiance::mxfp4_linear_pq", mutates_args=())
def mxfp4_linear_pq(x_fp8: torch.Tensor, x_scale: torch.Tensor, weight: torch.Tensor,
                    weight_scale: torch.Tensor, weight_ref: torch.Tensor,
                    allow_tiled: bool = True) -> torch.Tensor:
    """Pre-quantized entry (sly/mxfp4/radiance_mxfp4.py:825-860): (e4m3 [M, K], fp32 [M]) -> bf16
    [M, N]. x_fp8 is row-major, or fragment-tiled when a producer recorded it so (TiledHandoff;
    tiled M x K is an [M, K] view over padded storage, so the shape is M either way).
    allow_tiled=False skips the lookup, for callers that quantized row-major themselves."""
    STATS["calls_pq"] += 1
    _diag.report_stats(STATS)
    N, K = weight_ref.shape[0], weight_ref.shape[1]
    if x_fp8.dim() != 2 or x_fp8.shape[1] != K or not x_fp8.is_contiguous():
        raise RuntimeError(f"[radiance.mxfp4] x_fp8 {tuple(x_fp8.shape)} must be contiguous "
                           f"[M, {K}]")
    if x_fp8.dtype not in (torch.float8_e4m3fn, torch.uint8):
        raise RuntimeError(f"[radiance.mxfp4] x_fp8 must be float8_e4m3fn, got {x_fp8.dtype}")
    M = x_fp8.shape[0]
    xs = x_scale.reshape(-1)
    if xs.numel() != M or xs.dtype != torch.float32 or not xs.is_contiguous():
        raise RuntimeError(f"[radiance.mxfp4] x_scale must be {M} contiguous fp32 values")
    if allow_tiled and A_TILED_MIN_M and a_tiled_take(x_fp8, M, K):
        STATS["calls_tiled"] += 1
        out = _diag.new_out(M, N, x_fp8.device)
        _native.gemm_at(x_fp8.data_ptr(), xs.data_ptr(), weight.data_ptr(),
                        weight_scale.data_ptr(), out.data_ptr(), M, N, K, _stream())
        return _diag.returned(out)  # fragment-tiled q: the row-major check does not apply
    out = gemm(x_fp8, xs, weight, weight_scale, N, K, out=_diag.new_out(M, N, x_fp8.device))
    if _diag.enabled():
        _diag.after_call(STATS, x_fp8, xs, weight, weight_scale, out, N, K)
    return _diag.returned(out)


@mxfp4_linear_pq.register_fake
def _(x_fp8, x_scale, weight, weight_scale, weight_ref, allow_tiled=True):
    return torch.empty((x_fp8.shape[0], weight_ref.shape[0]), device=x_fp8.device,
                       dtype=torch.bfloat16)


@torch.library.custom_op("radiance::silu_mul_mxfp4_linear", mutates_args=())
def silu_mul_mxfp4_linear(gate_up: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor,
                          weight_ref: torch.Tensor) -> torch.Tensor:
    """The MLP's tail in one op: gate_up bf16 [M, 2K] -> the down projection [M, N] of
    silu(gate) * up, the same bits as radiance::silu_mul_quant followed by mxfp4_linear_pq (the
    reference's pair, sly/mxfp4/radiance_fused_norm.py:163-180 and sly/mxfp4/radiance_mxfp4.py:
    825-860). At M <= 2 one launch: the streaming GEMM's quantizing waves form and quantize the
    SiLU-and-mul stage while its weight waves stream; otherwise the producer and the GEMM."""
    STATS["calls_silu"] += 1
    _diag.report_stats(STATS)
    N, K = weight_ref.shape[0], weight_ref.shape[1]
    if gate_up.dim() != 2 or gate_up.shape[1] != 2 * K:
        raise RuntimeError(f"[radiance.mxfp4] gate_up {tuple(gate_up.shape)} does not match "
                           f"2K={2 * K}")
    if gate_up.dtype != torch.bfloat16:
        raise RuntimeError(f"[radiance.mxfp4] gate_up must be bf16, got {gate_up.dtype}")
    gate_up = gate_up.contiguous()
    M = gate_up.shape[0]
    out = _diag.new_out(M, N, gate_up.device)
    q = torch.empty((M, K), dtype=torch.float8_e4m3fn, device=gate_up.device)
    s = torch.empty((M,), dtype=torch.float32, device=gate_up.device)
    if M:
        _native.silu_mul_linear(gate_up.data_ptr(), q.data_ptr(), s.data_ptr(), weight.data_ptr(),
                                weight_scale.data_ptr(), out.data_ptr(), M, N, K, _stream())
    if _diag.enabled():
        def _quantized(gate_up=gate_up, M=M, K=K):
            # the SiLU-and-mul producer's (q, scale): the one-launch form keeps them in LDS
            q2 = torch.empty((M, K), dtype=torch.float8_e4m3fn, device=gate_up.device)
            s2 = torch.empty((M,), dtype=torch.float32, device=gate_up.device)
            _native.silu_mul_quant(gate_up.data_ptr(), q2.data_ptr(), s2.data_ptr(), M, K,
                                   _stream())
            return q2, s2
        _diag.after_call(STATS, _quantized, None, weight, weight_scale, out, N, K, x=gate_up)
    return _diag.returned(out)


@silu_mul_mxfp4_linear.register_fake
def _(gate_up, weight, weight_scale, weight_ref):
    return torch.empty((gate_up.shape[0], weight_ref.shape[0]), device=gate_up.device,
                       dtype=torch.bfloat16)


# --------------------------------------------------------------------------------------------
# The kernel plugin (vLLM MxFp4LinearKernel ABC)
# --------------------------------------------------------------------------------------------
def on_gfx950() -> bool:
    try:
        return torch.cuda.is_available() and \
            torch.cuda.get_device_properties(torch.cuda.current_device()).gcnArchName \
                .split(":")[0] == "gfx950"
    except Exception:
        return False


def layer_is_supported(layer, K: int) -> bool:
    """Load-time shape gate (sly/mxfp4/radiance_mxfp4.py:960-977): K a multiple of the MX block,
    weight [N, K/2] and weight_scale [N, K/32] in the checkpoint layout."""
    try:
        N = layer.weight.shape[0]
        return bool(K % 32 == 0 and layer.weight.dtype == torch.uint8
                    and layer.weight.shape[1] * 2 == K
                    and tuple(layer.weight_scale.shape) == (N, K // 32))
    except Exception:
        return False


def aiter_asm_fp4_enabled() -> bool:
    """True when vLLM routes MXFP4 through AITER's asm fp4 GEMM, which keeps its weights shuffled
    and its scales swizzled: a layer prepared for it is not a checkpoint layer this kernel can
    repack, so can_implement declines (sly/mxfp4/radiance_mxfp4.py:995-1004, :1032-1036).
    False when vLLM or its AITER hooks are absent."""
    try:
        from vllm._aiter_ops import rocm_aiter_ops
        return bool(rocm_aiter_ops.is_asm_fp4_gemm_dynamic_quant_enabled())
    except Exception:
        return False


def _base_classes():
    """vLLM's ABC and activation key when vLLM is importable, else local stand-ins with the same
    names (vllm.model_executor.kernels.linear.mxfp4.base, sly/mxfp4/radiance_mxfp4.py:1010-1014)."""
    try:
        from vllm.model_executor.kernels.linear.mxfp4.base import MxFp4LinearKernel
        from vllm.model_executor.layers.quantization.utils.quant_utils import kMxfp4Dynamic
        return MxFp4LinearKernel, kMxfp4Dynamic
    except Exception:
        class MxFp4LinearKernel:  # minimal stand-in: config holder, as vLLM's base class is
            def __init__(self, config=None, *args, **kwargs):
                self.config = config
        return MxFp4LinearKernel, ACTIVATION_QUANT_KEY


def _make_kernel_class():
    Base, quant_key = _base_classes()

    class RadianceMxfp4W4A8LinearKernel(Base):
        """MXFP4 weights x fp8 activations on gfx950 via the scaled-MFMA HIP kernels."""

        @classmethod
        def is_supported(cls, compute_capability=None):
            if not ENABLED:
                return False, "RADIANCE_MXFP4_W4A8 is not enabled"
            try:
                _native.lib()
            except Exception as e:  # noqa: BLE001
                return False, f"the gfx950 W4A8 library failed to load: {e}"
            if not on_gfx950():
                return False, "the radiance W4A8 MXFP4 kernels are built for gfx950 only"
            return True, None

        @classmethod
        def can_implement(cls, config):
            if getattr(config, "activation_quant_key", None) != quant_key:
                return False, "only supports MXFP4 dynamic activation"
            if aiter_asm_fp4_enabled():
                return False, "AITER's asm fp4 GEMM owns this layer's weight layout"
            return True, None

        def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
            """Repack the checkpoint weight into MFMA granules, in the same storage when the shape
            is aligned (N % 16 == 0, K % 512 == 0), and attach the layout descriptor. Refuses a
            layer it cannot serve rather than computing something wrong."""
            N, K = int(layer.weight.shape[0]), int(layer.weight.shape[1]) * 2
            if not layer_is_supported(layer, K):
                STATS["refused"] += 1
                raise RuntimeError(
                    f"[radiance.mxfp4] layer N={N} K={K} weight {tuple(layer.weight.shape)} "
                    f"{layer.weight.dtype} / weight_scale {tuple(layer.weight_scale.shape)} is not "
                    f"an MXFP4 checkpoint layer this kernel serves")
            ensure_scratch(layer.weight.device)
            wq, sq = repack_weights(layer.weight.data, layer.weight_scale.data)
            if wq.shape == layer.weight.shape and layer.weight.is_contiguous():
                layer.weight.data.copy_(wq)              # same storage: no allocator holes
            else:
                layer.weight = torch.nn.Parameter(wq, requires_grad=False)
            if sq.shape == layer.weight_scale.shape and layer.weight_scale.is_contiguous():
                layer.weight_scale.data.copy_(sq)
            else:
                layer.weight_scale = torch.nn.Parameter(sq, requires_grad=False)
            del wq, sq
            layer.radiance_wref = torch.nn.Parameter(layout_ref(N, K, layer.weight.device),
                                                     requires_grad=False)
            layer.radiance_w4a8_ok = True
            STATS["fast"] += 1

        def apply_weights(self, layer: torch.nn.Module, x, bias: torch.Tensor | None = None):
            if isinstance(x, tuple):
                x_fp8, x_scale = x
                y = torch.ops.radiance.mxfp4_linear_pq(
                    x_fp8, x_scale, layer.weight, layer.weight_scale, layer.radiance_wref)
            else:
                lead = x.shape[:-1]
                y = torch.ops.radiance.mxfp4_linear(
                    x.reshape(-1, x.shape[-1]), layer.weight, layer.weight_scale,
                    layer.radiance_wref)
                y = y.reshape(*lead, y.shape[-1])
            if bias is not None:
                y = y + bias
            return y

        def apply(self, layer: torch.nn.Module, x, bias: torch.Tensor | None = None):
            """LinearMethodBase.apply: the quant-method entry vLLM's Linear.forward calls."""
            return self.apply_weights(layer, x, bias)

    return RadianceMxfp4W4A8LinearKernel


_KERNEL_CLS = None


def kernel_class():
    """The plugin class, built once (sly/mxfp4/radiance_mxfp4.py:1223-1234)."""
    global _KERNEL_CLS
    if _KERNEL_CLS is None:
        _KERNEL_CLS = _make_kernel_class()
    return _KERNEL_CLS


def _is_mxfp4(args, kwargs) -> bool:
    q = kwargs.get("quantization", args[0] if args else None)
    return isinstance(q, str) and q.lower() == "mxfp4"


def register_with_vllm(platform=None) -> bool:
    """Put the plugin at the head of vLLM's MXFP4 kernel priority list, the one change
    sly/patch_quark_mxfp4.py:76-103 makes. The list is `_POSSIBLE_MXFP4_KERNELS[platform]` of
    vllm.model_executor.kernels.linear (the module init_mxfp4_linear_kernel reads it from), keyed
    by current_platform._enum unless `platform` is given. Idempotent: the class appears once, at
    index 0. Returns False when vLLM is not importable.

    The reference inserts the class after init_mxfp4_linear_kernel's --linear-backend filter
    (`possible = _resolve_backend_kernels(possible, "MXFP4")`), so the filter never drops it. An
    entry in the list alone would go through that filter, so the module's _resolve_backend_kernels
    is wrapped once as well: for the MXFP4 list, a filtered result that lost the plugin gets it back
    at its head, which is the reference's order; every other call passes through unchanged."""
    try:
        import vllm.model_executor.kernels.linear as registry
        if platform is None:
            from vllm.platforms import current_platform
            platform = current_platform._enum
    except Exception as e:  # noqa: BLE001
        sys.stderr.write(f"[radiance.mxfp4] vLLM not importable, plugin not registered: {e!r}\n")
        return False
    cls = kernel_class()
    kernels = registry._POSSIBLE_MXFP4_KERNELS.setdefault(platform, [])
    kernels[:] = [cls] + [k for k in kernels if k is not cls]
    resolve = getattr(registry, "_resolve_backend_kernels", None)
    if resolve is not None and not getattr(resolve, "_radiance_keeps_plugin", False):
        def _resolve_backend_kernels(possible, *args, **kwargs):
            out = resolve(possible, *args, **kwargs)
            if _is_mxfp4(args, kwargs) and cls in possible and cls not in out:
                out = [cls] + list(out)
            return out
        _resolve_backend_kernels._radiance_keeps_plugin = True
        _resolve_backend_kernels.__wrapped__ = resolve
        registry._resolve_backend_kernels = _resolve_backend_kernels
    return True
