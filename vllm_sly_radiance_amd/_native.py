"""ctypes binding of libw4a8_mxfp4.so (C ABI: include/w4a8_mxfp4.h).

The library is loaded after torch so that its libamdhip64.so.7 dependency binds to the HIP runtime
torch already mapped (same soname): one runtime, one set of streams. There is no fallback: a
missing or stale library raises, and so does every nonzero status (RuntimeError carrying
w4a8_last_error(), as the reference's pybind module raised RuntimeError from std::runtime_error,
sly/mxfp4/radiance_mxfp4_fp8.hip:1378-1385).
"""
from __future__ import annotations

import ctypes
import os
import threading

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libw4a8_mxfp4.so")
ABI_VERSION = 2
(KERNEL_AUTO, KERNEL_SKINNY, KERNEL_TILE, KERNEL_STREAM, KERNEL_RING, KERNEL_TILE_AT,
 KERNEL_RING_AT, KERNEL_BAND) = range(8)
Q_ROWS, Q_TILED = 0, 1          # layouts of a producer's q

_c = ctypes
_vp, _int, _long, _sz = _c.c_void_p, _c.c_int, _c.c_long, _c.c_size_t
_pint, _psz = _c.POINTER(_c.c_int), _c.POINTER(_c.c_size_t)

# name -> (restype, argtypes); the exported surface, checked against the header by the tests
SIGNATURES = {
    "w4a8_abi_version": (_int, []),
    "w4a8_last_error": (_c.c_char_p, []),
    "w4a8_layout_version": (_int, []),
    "w4a8_packed_bytes": (_int, [_int, _int, _psz, _psz]),
    "w4a8_quant_per_token": (_int, [_vp, _long, _vp, _vp, _int, _int, _vp]),
    "w4a8_repack": (_int, [_vp, _vp, _vp, _vp, _int, _int, _vp]),
    "w4a8_set_scratch": (_int, [_vp, _sz, _vp, _sz]),
    "w4a8_gemm": (_int, [_vp, _vp, _vp, _vp, _vp, _int, _int, _int, _vp]),
    "w4a8_gemm_at": (_int, [_vp, _vp, _vp, _vp, _vp, _int, _int, _int, _vp]),
    "w4a8_tiled_bytes": (_int, [_int, _int, _psz]),
    "w4a8_plan": (_int, [_int, _int, _int, _pint, _pint, _pint]),
    "w4a8_gemm_planned": (_int, [_vp, _vp, _vp, _vp, _vp, _int, _int, _int, _int, _int, _int,
                                 _vp]),
    "w4a8_gemm_noalloc": (_int, [_vp, _vp, _vp, _vp, _vp, _int, _int, _int, _int, _int, _int,
                                 _vp]),
    "w4a8_variant_count": (_int, [_int]),
    "w4a8_variant_info": (_int, [_int, _int, _pint, _pint, _pint, _pint]),
    "w4a8_tile_config": (_int, [_int, _pint, _pint, _pint, _pint, _pint]),
    "w4a8_variant_serves": (_int, [_int, _int, _int, _int, _int, _int]),
    "w4a8_scratch_bytes": (_int, [_int, _int, _int, _psz, _psz]),
    "w4a8_workspace_bytes": (_int, [_int, _int, _psz, _psz]),
    "w4a8_linear": (_int, [_vp, _long, _vp, _vp, _vp, _vp, _vp, _int, _int, _int, _vp]),
    "w4a8_linear_fused": (_int, [_int, _int, _int, _long]),
    "w4a8_add_rms_quant": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _int, _int, _c.c_float, _vp,
                                  _int]),
    "w4a8_silu_mul_quant": (_int, [_vp, _vp, _vp, _int, _int, _vp, _int]),
    "w4a8_silu_mul": (_int, [_vp, _vp, _int, _int, _vp]),
    "w4a8_silu_mul_linear": (_int, [_vp, _vp, _vp, _vp, _vp, _vp, _int, _int, _int, _vp]),
    "w4a8_silu_mul_linear_fused": (_int, [_int, _int, _int]),
    "w4a8_gdn_norm_quant": (_int, [_vp, _vp, _long, _vp, _vp, _vp, _int, _int, _c.c_float, _vp,
                                   _int]),
    "w4a8_mfma_probe": (_int, [_int, _vp, _int, _int, _c.POINTER(_c.c_double), _vp]),
    "w4a8_silu_f32": (_int, [_vp, _vp, _int, _vp]),
    "w4a8_read_probe": (_int, [_vp, _long, _vp, _vp]),
    "w4a8_read_probe_variants": (_int, []),
    "w4a8_read_probe_variant_info": (_int, [_int, _pint, _pint, _pint, _pint]),
    "w4a8_read_probe_shape": (_int, [_vp, _long, _vp, _int, _int, _vp]),
    "w4a8_stream_load_probe": (_int, [_vp, _vp, _vp, _vp, _int, _int, _int, _int, _vp, _vp]),
    "w4a8_mfma_tile": (_int, [_vp, _vp, _vp, _vp, _vp, _int, _vp]),
}

_lock = threading.Lock()
_lib = None


def load_cdll(path: str = LIB_PATH) -> ctypes.CDLL:
    """dlopen the library and declare every signature (no GPU needed)."""
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built: run __graft_entry__.build() "
                           "(hipcc --offload-arch=gfx950) first")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    if lib.w4a8_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{path}: ABI {lib.w4a8_abi_version()} != expected {ABI_VERSION}")
    return lib


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                import torch  # noqa: F401  (bind to torch's HIP runtime before dlopen)
                _lib = load_cdll()
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        raise RuntimeError("[radiance.mxfp4] " + lib().w4a8_last_error().decode(errors="replace"))


# ---- thin typed wrappers over raw device pointers -------------------------------------------
def quant_per_token(x_ptr, ldx, q_ptr, s_ptr, M, K, stream):
    check(lib().w4a8_quant_per_token(x_ptr, ldx, q_ptr, s_ptr, M, K, stream))


def repack(w_ptr, ws_ptr, wq_ptr, sq_ptr, N, K, stream):
    check(lib().w4a8_repack(w_ptr, ws_ptr, wq_ptr, sq_ptr, N, K, stream))


def gemm(a_ptr, as_ptr, wq_ptr, sq_ptr, c_ptr, M, N, K, stream, kernel=KERNEL_AUTO, variant=-1,
         split_k=0):
    check(lib().w4a8_gemm_planned(a_ptr, as_ptr, wq_ptr, sq_ptr, c_ptr, M, N, K, kernel, variant,
                                  split_k, stream))


def gemm_noalloc(a_ptr, as_ptr, wq_ptr, sq_ptr, c_ptr, M, N, K, stream, kernel=KERNEL_AUTO,
                 variant=-1, split_k=0):
    """gemm() on the library's static scratch: allocates nothing, needs no set_scratch."""
    check(lib().w4a8_gemm_noalloc(a_ptr, as_ptr, wq_ptr, sq_ptr, c_ptr, M, N, K, kernel, variant,
                                  split_k, stream))


def gemm_at(a_ptr, as_ptr, wq_ptr, sq_ptr, c_ptr, M, N, K, stream):
    """The GEMM on fragment-tiled activations (a producer's q written with Q_TILED)."""
    check(lib().w4a8_gemm_at(a_ptr, as_ptr, wq_ptr, sq_ptr, c_ptr, M, N, K, stream))


def variant_serves(kernel, variant, M, N, K, split_k=1) -> bool:
    """Does a forced plan (kernel, variant, split_k) serve this shape (no launch)."""
    r = lib().w4a8_variant_serves(kernel, variant, M, N, K, split_k)
    if r < 0:
        check(1)
    return bool(r)


def tiled_bytes(M: int, K: int) -> int:
    n = _sz()
    check(lib().w4a8_tiled_bytes(M, K, _c.byref(n)))
    return n.value


def linear(x_ptr, ldx, q_ptr, s_ptr, wq_ptr, sq_ptr, c_ptr, M, N, K, stream):
    check(lib().w4a8_linear(x_ptr, ldx, q_ptr, s_ptr, wq_ptr, sq_ptr, c_ptr, M, N, K, stream))


def linear_fused(M: int, N: int, K: int, ldx: int) -> bool:
    """Does linear() run this shape as one launch (quantizer inside the streaming GEMM)."""
    r = lib().w4a8_linear_fused(M, N, K, ldx)
    if r < 0:
        check(1)
    return bool(r)


def add_rms_quant(y_ptr, res_ptr, w_ptr, q_ptr, s_ptr, res_out_ptr, M, K, eps, stream,
                  q_layout=Q_ROWS):
    check(lib().w4a8_add_rms_quant(y_ptr, res_ptr, w_ptr, q_ptr, s_ptr, res_out_ptr, M, K, eps,
                                   stream, q_layout))


def silu_mul_quant(gu_ptr, q_ptr, s_ptr, M, N, stream, q_layout=Q_ROWS):
    check(lib().w4a8_silu_mul_quant(gu_ptr, q_ptr, s_ptr, M, N, stream, q_layout))


def silu_mul(gu_ptr, out_ptr, M, N, stream):
    check(lib().w4a8_silu_mul(gu_ptr, out_ptr, M, N, stream))


def silu_mul_linear(gu_ptr, q_ptr, s_ptr, wq_ptr, sq_ptr, c_ptr, M, N, K, stream):
    check(lib().w4a8_silu_mul_linear(gu_ptr, q_ptr, s_ptr, wq_ptr, sq_ptr, c_ptr, M, N, K, stream))


def silu_mul_linear_fused(M: int, N: int, K: int) -> bool:
    """Does silu_mul_linear() run this shape as one launch (SiLU-mul and quantizer inside the
    streaming GEMM)."""
    r = lib().w4a8_silu_mul_linear_fused(M, N, K)
    if r < 0:
        check(1)
    return bool(r)


def gdn_norm_quant(x_ptr, z_ptr, z_stride, w_ptr, q_ptr, s_ptr, M, N, eps, stream,
                   q_layout=Q_ROWS):
    check(lib().w4a8_gdn_norm_quant(x_ptr, z_ptr, z_stride, w_ptr, q_ptr, s_ptr, M, N, eps,
                                    stream, q_layout))


def set_scratch(partial_ptr, partial_bytes, counter_ptr, counter_bytes):
    check(lib().w4a8_set_scratch(partial_ptr, partial_bytes, counter_ptr, counter_bytes))


def packed_bytes(N: int, K: int):
    a, b = _sz(), _sz()
    check(lib().w4a8_packed_bytes(N, K, _c.byref(a), _c.byref(b)))
    return a.value, b.value


def plan(M: int, N: int, K: int):
    k, v, s = _int(), _int(), _int()
    check(lib().w4a8_plan(M, N, K, _c.byref(k), _c.byref(v), _c.byref(s)))
    return k.value, v.value, s.value


def variants(kernel: int):
    n = lib().w4a8_variant_count(kernel)
    if n < 0:
        check(1)
    out = []
    for v in range(n):
        p = [_int() for _ in range(4)]
        check(lib().w4a8_variant_info(kernel, v, *[_c.byref(x) for x in p]))
        out.append(tuple(x.value for x in p))
    return out


def tile_config(variant: int) -> dict:
    """A macro-tile variant's workgroup tile, pipeline depth, waves and LDS bytes."""
    p = [_int() for _ in range(5)]
    check(lib().w4a8_tile_config(variant, *[_c.byref(x) for x in p]))
    return dict(zip(("bm", "bn", "stages", "waves", "lds"), (x.value for x in p)))


def tile_stages(variant: int) -> int:
    return tile_config(variant)["stages"]


def scratch_bytes(variant: int, N: int, split_k: int):
    a, b = _sz(), _sz()
    check(lib().w4a8_scratch_bytes(variant, N, split_k, _c.byref(a), _c.byref(b)))
    return a.value, b.value


def workspace_bytes(max_m: int, max_n: int):
    """(partial bytes, counter bytes) the automatic plan may use for M <= max_m, N <= max_n."""
    a, b = _sz(), _sz()
    check(lib().w4a8_workspace_bytes(max_m, max_n, _c.byref(a), _c.byref(b)))
    return a.value, b.value


def silu_f32(x_ptr, y_ptr, n, stream) -> None:
    """The producers' fp32 silu of n bf16 values (n % 8 == 0), unrounded (a diagnostic)."""
    check(lib().w4a8_silu_f32(x_ptr, y_ptr, n, stream))


def read_probe(buf_ptr, nbytes, out_ptr, stream) -> None:
    check(lib().w4a8_read_probe(buf_ptr, nbytes, out_ptr, stream))


def read_probe_variants():
    """[(waves, KiB per wave, loads in flight per wave, non-temporal)] of the shape probe."""
    out = []
    for v in range(lib().w4a8_read_probe_variants()):
        p = [_c.c_int() for _ in range(4)]
        check(lib().w4a8_read_probe_variant_info(v, *[_c.byref(x) for x in p]))
        out.append(tuple(x.value for x in p))
    return out


def read_probe_shape(buf_ptr, nbytes, out_ptr, blocks, variant, stream) -> None:
    check(lib().w4a8_read_probe_shape(buf_ptr, nbytes, out_ptr, blocks, variant, stream))


# parts of w4a8_stream_load_probe: the weight granules; and the scale dwords; and the activation
# fragments with the token scales (every load of the streaming GEMM)
STREAM_LOADS_WEIGHTS, STREAM_LOADS_SCALES, STREAM_LOADS_ALL = 1, 3, 7


def stream_load_probe(a_ptr, as_ptr, wq_ptr, sq_ptr, M, N, K, parts, out_ptr, stream) -> None:
    check(lib().w4a8_stream_load_probe(a_ptr, as_ptr, wq_ptr, sq_ptr, M, N, K, parts, out_ptr,
                                       stream))


def mfma_probe(shape, out_ptr, blocks, iters, stream) -> float:
    """Launch the MFMA throughput probe; returns the FLOP it performs."""
    f = _c.c_double()
    check(lib().w4a8_mfma_probe(shape, out_ptr, blocks, iters, _c.byref(f), stream))
    return f.value


def mfma_tile(a_ptr, b_ptr, sa_ptr, sb_ptr, d_ptr, count, stream):
    check(lib().w4a8_mfma_tile(a_ptr, b_ptr, sa_ptr, sb_ptr, d_ptr, count, stream))
