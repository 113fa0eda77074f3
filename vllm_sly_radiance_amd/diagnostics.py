"""In-situ diagnostics of the linear path, off by default and free when off.

The reference's op body carries these, and they keep its switch names:
  RADIANCE_MXFP4_CHECKALL="N:K,N:K"  every call of the listed shapes with M <= CHECK_MAX_M
                                     (RADIANCE_MXFP4_CHECK_MAX_M, default 128) is compared with an
                                     fp32 dequant-then-matmul of the same e4m3 activations and the
                                     layer's repacked weights, computed by torch on the device; a
                                     rel-L2 above 0.02 counts as wrong and is reported (the first
                                     8), the others are reported at a shape's 1st and 64th call
                                     (sly/mxfp4/radiance_mxfp4.py:470-477, :761-785).
  RADIANCE_MXFP4_MHIST=1             every distinct (N, K, M) is reported once, with the plan the
                                     library takes for it (:500-502, :755-760).
  RADIANCE_MXFP4_CHECKX=1            each distinct (N, K, M), the first 60, reports the health of
                                     its input and output: mean and max magnitude and non-finite
                                     counts (:468-469, :786-799)
  RADIANCE_MXFP4_SYNC=1 / 2          synchronize the op's stream / the whole device after every
                                     call, to tell ordering faults from wrong values (:425-431,
                                     :800-803)
  RADIANCE_MXFP4_SANITIZE=1          zero NaN and inf in the bf16 activations before they are
                                     quantized (a NaN otherwise makes its row's scale, and so the
                                     whole output row, NaN; :450-466, :715-716)
  RADIANCE_MXFP4_DEBUG=1             each distinct (N, K, M) with M <= 128, the first 40, is compared
                                     once with the same exact fp32 product and reported ok or
                                     wrong (:557-577, :804-805)
  RADIANCE_MXFP4_CLONE=1             the op returns a copy of its output buffer (:433-436, :816)
  RADIANCE_MXFP4_PADOUT=n            the output is allocated inside a slab with n spare bf16
                                     elements before and after it, so nothing live is adjacent
                                     (:437-442, :733-736)
  report_stats()                     the one-shot tally of layers on the HIP kernel and layers
                                     refused at load (:941-957). It is called from op bodies only:
                                     they are opaque to dynamo, so a stderr write there cannot
                                     break a compiled graph.
Reports go to stderr. A check synchronizes the stream, so it is skipped while the stream is being
captured into a graph. The check's reference never replaces the kernel's output.
"""
from __future__ import annotations

import os
import sys

import torch

from . import _native


def parse_shapes(spec: str):
    """"17408:5120,5120:8704" -> {(17408, 5120), (5120, 8704)}; empty -> None."""
    spec = spec.strip()
    if not spec:
        return None
    out = set()
    for pair in spec.split(","):
        if pair.strip():
            n, k = pair.split(":")
            out.add((int(n), int(k)))
    return out or None


CHECK_ALL = parse_shapes(os.environ.get("RADIANCE_MXFP4_CHECKALL", ""))
CHECK_MAX_M = int(os.environ.get("RADIANCE_MXFP4_CHECK_MAX_M", "128"))
MHIST = os.environ.get("RADIANCE_MXFP4_MHIST", "0") == "1"
CHECK_X = os.environ.get("RADIANCE_MXFP4_CHECKX", "0") == "1"
SYNC = os.environ.get("RADIANCE_MXFP4_SYNC", "0")
SANITIZE_X = os.environ.get("RADIANCE_MXFP4_SANITIZE", "0") == "1"
DEBUG = os.environ.get("RADIANCE_MXFP4_DEBUG", "0") == "1"
CLONE_OUT = os.environ.get("RADIANCE_MXFP4_CLONE", "0") == "1"
PAD_OUT = int(os.environ.get("RADIANCE_MXFP4_PADOUT", "0"))
CHECK_X_MAX = 60
DEBUG_MAX = 40
WRONG_REL = 0.02

KERNEL_NAMES = {_native.KERNEL_SKINNY: "skinny", _native.KERNEL_TILE: "tile",
                _native.KERNEL_STREAM: "stream", _native.KERNEL_RING: "ring",
                _native.KERNEL_TILE_AT: "tile_at", _native.KERNEL_RING_AT: "ring_at",
                _native.KERNEL_BAND: "band"}

_seen: set = set()
_reported = [False]

# e2m1 code -> value, bit 3 the sign
_E2M1 = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0)


def unrepack(wq: torch.Tensor, sq: torch.Tensor, N: int, K: int):
    """Granules and scale dwords back to the checkpoint layout: (uint8 [N, K/2], uint8 [N, K/32]).

    Granule (n-tile t, k-tile j) holds lane l's 16 bytes at ((t KT + j) 64 + l) 16: column
    16 t + l % 16, 32-element block 4 j + l / 16, nibbles in checkpoint order. The scale dword of
    lane l for k-group g sits at ((t KG + g) 64 + l) 4; its byte b is block 4 (4 g + b) + l / 16
    of column 16 t + l % 16."""
    Np, Kp = -(-N // 16) * 16, -(-K // 512) * 512
    NT, KT, KG = Np // 16, Kp // 128, Kp // 512
    w = wq.reshape(NT, KT, 4, 16, 16).permute(0, 3, 1, 2, 4).reshape(Np, Kp // 2)
    s = sq.reshape(NT, KG, 4, 16, 4).permute(0, 3, 1, 4, 2).reshape(Np, Kp // 32)
    return w[:N, :K // 2], s[:N, :K // 32]


def exact_linear(x_fp8: torch.Tensor, x_scale: torch.Tensor, wq: torch.Tensor, sq: torch.Tensor,
                 N: int, K: int, chunk: int = 2048) -> torch.Tensor:
    """fp32 [M, N]: the e4m3 activations times their token scales, times the dequantized weight
    (e2m1 x 2^(e - 127) per 32-element block), one fp32 matmul per chunk of columns so that the
    dequantized weight never exists whole next to a loaded model."""
    w, ws = unrepack(wq, sq, N, K)
    table = torch.tensor(_E2M1, dtype=torch.float32, device=wq.device)
    xr = x_fp8.view(torch.float8_e4m3fn).float() * x_scale.reshape(-1, 1).float()
    outs = []
    for a in range(0, N, chunk):
        b = min(a + chunk, N)
        wc = w[a:b]
        codes = torch.stack([wc & 0x0F, wc >> 4], dim=-1).reshape(b - a, K).long()
        scale = torch.pow(2.0, ws[a:b].float() - 127.0).repeat_interleave(32, dim=1)
        outs.append(xr @ (table[codes] * scale).T)
    return torch.cat(outs, dim=1)


def report_stats(stats: dict) -> None:
    """The one-shot tally (sly/mxfp4/radiance_mxfp4.py:945-957)."""
    if _reported[0]:
        return
    _reported[0] = True
    n = stats["fast"] + stats["refused"]
    sys.stderr.write(f"[radiance.mxfp4] linear layers: {stats['fast']}/{n} on the gfx950 W4A8 "
                     f"kernels, {stats['refused']} refused at load (not a checkpoint layout "
                     f"they serve)\n")
    sys.stderr.flush()


def enabled() -> bool:
    return MHIST or CHECK_ALL is not None or CHECK_X or DEBUG or SYNC in ("1", "2")


def new_out(M: int, N: int, device) -> torch.Tensor:
    """The op's bf16 [M, N] output: torch.empty, or with RADIANCE_MXFP4_PADOUT=n a view into a
    slab holding n spare elements on each side (the kernels store through any 2-byte alignment)."""
    if PAD_OUT <= 0:
        return torch.empty((M, N), dtype=torch.bfloat16, device=device)
    slab = torch.empty(M * N + 2 * PAD_OUT, dtype=torch.bfloat16, device=device)
    return slab[PAD_OUT:PAD_OUT + M * N].view(M, N)


def returned(out: torch.Tensor) -> torch.Tensor:
    """What the op hands back: its output, or a copy of it with RADIANCE_MXFP4_CLONE=1."""
    return out.clone() if CLONE_OUT else out


def sanitize(x: torch.Tensor) -> torch.Tensor:
    """x with NaN and inf zeroed when RADIANCE_MXFP4_SANITIZE=1 (a new tensor), else x itself."""
    if not SANITIZE_X:
        return x
    return torch.nan_to_num(x, nan=0.0, posinf=0.0, neginf=0.0)


def _health(x: torch.Tensor | None, out: torch.Tensor, N: int, K: int) -> None:
    M = int(out.shape[0])
    key = ("x", N, K, M)
    if key in _seen or sum(1 for k in _seen if k[0] == "x") >= CHECK_X_MAX:
        return
    _seen.add(key)
    of = out.float()
    head = f"[radiance.mxfp4.x] N={N} K={K} M={M} "
    if x is not None:
        xf = x.float()
        head += (f"|x|={xf.abs().mean().item():.5f} xmax={xf.abs().max().item():.5f} "
                 f"x_nonfin={int((~torch.isfinite(xf)).sum().item())} | ")
    sys.stderr.write(head + f"|out|={of.abs().mean().item():.5f} "
                     f"outmax={of.abs().max().item():.5f} "
                     f"out_nonfin={int((~torch.isfinite(of)).sum().item())}\n")
    sys.stderr.flush()


def after_call(stats: dict, x_fp8, x_scale, wq, sq, out, N: int, K: int, x=None) -> None:
    """Run the enabled diagnostics on one finished call. x_fp8 / x_scale are the call's e4m3
    activations and token scales, or a callable returning them (computed only if a check runs);
    x is the bf16 input where the op has one (for the health report)."""
    M = int(out.shape[0])
    capturing = torch.cuda.is_current_stream_capturing()
    if SYNC == "1" and not capturing:
        torch.cuda.current_stream().synchronize()
    elif SYNC == "2" and not capturing:
        torch.cuda.synchronize()
    if CHECK_X and not capturing and M:
        _health(x, out, N, K)
    if MHIST and ("m", N, K, M) not in _seen:
        _seen.add(("m", N, K, M))
        k, v, s = _native.plan(M, N, K) if M else (0, -1, 1)
        sys.stderr.write(f"[radiance.mxfp4.mhist] N={N} K={K} M={M} "
                         f"plan={KERNEL_NAMES.get(k, k)} variant={v} split_k={s}\n")
        sys.stderr.flush()
    debug = (DEBUG and not capturing and 0 < M <= 128 and ("d", N, K, M) not in _seen
             and sum(1 for k in _seen if k[0] == "d") < DEBUG_MAX)
    check = not (CHECK_ALL is None or (N, K) not in CHECK_ALL or M == 0 or M > CHECK_MAX_M
                 or capturing)
    if not (debug or check):
        return
    if callable(x_fp8):
        x_fp8, x_scale = x_fp8()
    ref = exact_linear(x_fp8, x_scale, wq, sq, N, K)
    if debug:
        _seen.add(("d", N, K, M))
        rel = ((out.float() - ref).norm() / ref.norm().clamp_min(1e-9)).item()
        sys.stderr.write(f"[radiance.mxfp4.exact] N={N} K={K} M={M} rel_vs_fp32={rel:.5f} "
                         f"|ours|={out.float().abs().mean().item():.5f} "
                         f"|ref|={ref.abs().mean().item():.5f} "
                         f"{'ok' if rel <= WRONG_REL else '**WRONG**'}\n")
        sys.stderr.flush()
    if not check:
        return
    rel = ((out.float() - ref).norm() / ref.norm().clamp_min(1e-9)).item()
    stats["checked"] = stats.get("checked", 0) + 1
    if not rel <= WRONG_REL:                                 # NaN counts as wrong
        stats["wrong"] = stats.get("wrong", 0) + 1
        if stats["wrong"] <= 8:
            of = out.float()
            sys.stderr.write(f"[radiance.mxfp4.all] **WRONG** call#{stats['checked']} N={N} K={K} "
                             f"M={M} rel={rel:.4f} |ours|={of.abs().mean().item():.5f} "
                             f"|ref|={ref.abs().mean().item():.5f} "
                             f"out_nonfinite={int((~torch.isfinite(of)).sum().item())}\n")
    else:
        key = ("seen", N, K)
        stats[key] = stats.get(key, 0) + 1
        if stats[key] in (1, 64):
            sys.stderr.write(f"[radiance.mxfp4.all] ok N={N} K={K} M={M} call#{stats[key]} "
                             f"rel={rel:.5f} (wrong so far: {stats.get('wrong', 0)})\n")
    sys.stderr.flush()
