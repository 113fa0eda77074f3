"""The C-ABI library on the CPU: it loads, exports every symbol include/w4a8_mxfp4.h declares, and
rejects bad arguments before touching a GPU (no compute call is made here)."""
import ctypes
import os
import re
import subprocess

import pytest

from vllm_sly_radiance_amd import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "w4a8_mxfp4.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(w4a8_\w+)\s*\(", src, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_native.LIB_PATH):
        pytest.fail(f"{_native.LIB_PATH} missing: run __graft_entry__.build() first")
    return _native.load_cdll()


def test_header_declares_the_bound_surface():
    assert declared_functions() == sorted(_native.SIGNATURES)


def test_every_declared_symbol_is_exported(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", _native.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    missing = [f for f in declared_functions() if f not in exported]
    assert not missing, missing
    # nothing but the C ABI leaks out (C++ internals stay hidden)
    extra = sorted(s for s in exported if not s.startswith("w4a8_") and not s.startswith("_"))
    assert not extra, extra


def test_library_is_built_for_gfx950_only(lib, tmp_path):
    # --offloading extracts the device images next to its input: work on a copy in tmp_path
    copy = tmp_path / "lib.so"
    copy.write_bytes(open(_native.LIB_PATH, "rb").read())
    out = subprocess.run(["/opt/rocm/llvm/bin/llvm-objdump", "--offloading", str(copy)],
                         capture_output=True, text=True, cwd=tmp_path)
    if out.returncode != 0:
        pytest.skip("llvm-objdump --offloading unavailable")
    arches = set(re.findall(r"amdhsa--(gfx\w+)", out.stdout))
    assert arches == {"gfx950"}, arches


def test_abi_and_layout_version(lib):
    assert lib.w4a8_abi_version() == _native.ABI_VERSION
    assert lib.w4a8_layout_version() == 1


def test_packed_bytes(lib):
    a, b = ctypes.c_size_t(), ctypes.c_size_t()
    assert lib.w4a8_packed_bytes(17408, 5120, ctypes.byref(a), ctypes.byref(b)) == 0
    assert (a.value, b.value) == (17408 * 5120 // 2, 17408 * 5120 // 32)
    assert lib.w4a8_packed_bytes(33, 96, ctypes.byref(a), ctypes.byref(b)) == 0
    assert (a.value, b.value) == (48 * 512 // 2, 48 * 512 // 32)
    assert lib.w4a8_packed_bytes(16, 48, ctypes.byref(a), ctypes.byref(b)) != 0
    assert b"multiple of 32" in lib.w4a8_last_error()


@pytest.mark.parametrize("M,N,K,msg", [(8, 5120, 5000, b"multiple of the 32-element"),
                                       (-1, 16, 128, b"M >= 0"), (8, 0, 128, b"N > 0")])
def test_gemm_rejects_bad_shapes_before_launch(lib, M, N, K, msg):
    rc = lib.w4a8_gemm(None, None, None, None, None, M, N, K, None)
    assert rc == 1 and msg in lib.w4a8_last_error()


def test_gemm_rejects_null_and_misaligned_pointers(lib):
    assert lib.w4a8_gemm(None, None, None, None, None, 8, 16, 128, None) == 1
    assert b"null pointer" in lib.w4a8_last_error()
    rc = lib.w4a8_gemm(4096 + 8, 4096, 4096, 4096, 4096, 8, 16, 128, None)
    assert rc == 1 and b"misaligned" in lib.w4a8_last_error()


def test_gemm_with_m_zero_is_a_no_op(lib):
    assert lib.w4a8_gemm(None, None, None, None, None, 0, 16, 128, None) == 0


def test_planned_rejects_unknown_kernel_and_variant(lib):
    p = 1 << 20
    assert lib.w4a8_gemm_planned(p, p, p, p, p, 8, 16, 128, 8, 0, 1, None) == 1
    assert b"unknown kernel" in lib.w4a8_last_error()
    assert lib.w4a8_variant_serves(8, 0, 8, 16, 128, 1) == -1
    # the band kernel (7): a variant index past its table, and one that does not serve the shape
    assert lib.w4a8_gemm_planned(p, p, p, p, p, 32, 16, 128, 7, 999, 1, None) == 1
    assert b"out of range" in lib.w4a8_last_error()
    assert lib.w4a8_variant_serves(7, 999, 32, 5120, 5120, 1) == 0
    assert lib.w4a8_gemm_planned(p, p, p, p, p, 8, 16, 128, 1, 999, 1, None) == 1
    assert b"out of range" in lib.w4a8_last_error()
    # a skinny variant refuses an M it does not cover
    assert lib.w4a8_gemm_planned(p, p, p, p, p, 40, 16, 128, 1, 0, 1, None) == 1
    assert b"covers M <=" in lib.w4a8_last_error()


def test_split_k_without_scratch_is_refused(lib):
    p = 1 << 20
    assert lib.w4a8_set_scratch(None, 0, None, 0) in (0, 3)   # 3: no HIP device on this host
    rc = lib.w4a8_gemm_planned(p, p, p, p, p, 8, 16, 4096, 1, 0, 4, None)
    assert rc == 2 and b"w4a8_set_scratch" in lib.w4a8_last_error()


def test_plan_bands(lib):
    k, v, s = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    # M <= 16: the streaming family when a wave's run and the LDS staging fit, else skinny; above
    # M = 16 the macro-tile family (the ring kernel only when forced).
    # N=17408 K=8704 would need 43-granule runs, past the largest stream variant; K=640 has fewer
    # k-tiles per n-tile than the smallest run.
    for M, N, K, kernel in [(1, 17408, 5120, 3), (8, 17408, 5120, 3), (16, 17408, 5120, 3),
                            (8, 5120, 8704, 3), (8, 17408, 8704, 1), (8, 33, 640, 1),
                            (17, 17408, 5120, 2), (64, 17408, 5120, 2), (65, 17408, 5120, 2),
                            (17, 5120, 6144, 2), (20, 5120, 8704, 2), (21, 5120, 8704, 2),
                            (20, 10240, 5120, 2), (17, 1024, 6144, 2), (20, 10256, 5120, 2),
                            (4096, 17408, 5120, 2)]:
        assert lib.w4a8_plan(M, N, K, ctypes.byref(k), ctypes.byref(v), ctypes.byref(s)) == 0
        assert (M, N, K, k.value) == (M, N, K, kernel) and v.value >= 0 and s.value >= 1
    assert lib.w4a8_plan(8, 17408, 5000, ctypes.byref(k), ctypes.byref(v), ctypes.byref(s)) == 1


@pytest.mark.parametrize("M,N,K,band_nt", [
    (33, 17408, 5120, 5), (40, 17408, 5120, 5), (48, 17408, 5120, 5), (48, 10240, 5120, 3),
    (33, 10240, 5120, 3), (32, 17408, 5120, None), (49, 17408, 5120, None), (64, 10240, 5120, None),
    (48, 5120, 8704, None), (48, 5120, 6144, None), (40, 8192, 5120, 2)])
def test_plan_band_kernel_between_33_and_48_tokens(lib, M, N, K, band_nt):
    """The band kernel (weight waves + activation waves) is the plan for 33..48 tokens on shapes of
    at least 8192 columns, with 48-token fragments and the fewest n-tiles per workgroup that cover
    the shape in one round; elsewhere in the band the macro tiles."""
    k, v, s = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    assert lib.w4a8_plan(M, N, K, ctypes.byref(k), ctypes.byref(v), ctypes.byref(s)) == 0
    if band_nt is None:
        assert k.value == _native.KERNEL_TILE
        return
    assert (k.value, s.value) == (_native.KERNEL_BAND, 1)
    mf, nt = _native.variants(_native.KERNEL_BAND)[v.value][:2]
    assert (mf, nt) == (3, band_nt)
    assert lib.w4a8_variant_serves(_native.KERNEL_BAND, v.value, M, N, K, 1) == 1


def test_one_launch_linear_where_it_pays(lib):
    """w4a8_linear runs as one launch (quantizing waves beside the streaming GEMM's weight waves)
    at M <= 2, and up to M = 4 where a workgroup holds 3 or more n-tiles or a quantizing wave
    handles at most 4 row chunks per lane (o_proj's 4-wave plan leaves 12 quantizing waves; down's
    6-wave plan leaves 10, 7 chunks per lane at M = 3..4); never on 16-wave variants (no room for
    the quantizing waves), never for rows that are not 16-byte chunks."""
    f = lib.w4a8_linear_fused
    for N, K, up_to in [(17408, 5120, 4), (10240, 5120, 4), (5120, 6144, 4), (5120, 8704, 2),
                        (5120, 5120, 4), (2048, 1024, 0), (1040, 512, 0)]:
        assert [f(M, N, K, K) for M in range(1, 10)] == [int(M <= up_to) for M in range(1, 10)], \
            (N, K)
    assert f(1, 17408, 5120, 5120 + 72) == 1
    assert f(1, 17408, 5120, 5120 + 4) == 0                # rows not whole 16-byte chunks
    assert f(1, 17408, 5000, 5000) == -1                   # K not a multiple of 32: an error
    assert f(1, 17408, 8704, 8704) == 0                    # no stream plan (skinny)
    assert f(0, 17408, 5120, 5120) == 0 and f(1, 17408, 5120, 5119) == 0


@pytest.mark.parametrize("M,N,K,tile", [
    # decode band above 16 tokens: 32 tokens tall and as narrow as keeps the workgroups within
    # one per CU (256 CUs); above 32 tokens 32 x 64 over both halves when that fits, else 64 x 64,
    # 64 x 96, 64 x 128
    (17, 5120, 6144, (32, 32)), (24, 5120, 8704, (32, 32)), (32, 10240, 5120, (32, 64)),
    (32, 17408, 5120, (32, 96)), (32, 65536, 5120, (32, 128)),
    (33, 5120, 6144, (32, 64)), (64, 17408, 5120, (64, 96)), (64, 5120, 8704, (32, 64)),
    (64, 10240, 5120, (64, 64)), (64, 65536, 5120, (64, 128)),
    # 64 < M <= 1024: the candidate with the least predicted time (tiles per CU x area / rate);
    # these are the measured-fastest variants at those points on MI355X
    (65, 10240, 5120, (32, 128)), (128, 10240, 5120, (64, 128)), (384, 10240, 5120, (128, 128)),
    (512, 10240, 5120, (256, 128)), (1024, 10240, 5120, (256, 160)),
    (128, 5120, 6144, (32, 128)), (384, 5120, 8704, (64, 128)), (768, 5120, 8704, (128, 128)),
    (1024, 5120, 8704, (256, 128)),
    (96, 17408, 5120, (128, 128)), (192, 17408, 5120, (64, 128)), (256, 17408, 5120, (256, 128)),
    (512, 17408, 5120, (256, 160)), (768, 17408, 5120, (256, 256)), (1024, 17408, 5120, (256, 160)),
    # M > 1024: the candidate (256 x 128, 256 x 160, 256 x 256, 128 x 256) whose rounds of
    # one-per-CU workgroups, with a ragged last round split off where the path splits it, take
    # the least predicted time
    (1280, 10240, 5120, (256, 256)), (1280, 5120, 6144, (256, 128)),
    (2048, 5120, 6144, (256, 160)), (2560, 5120, 8704, (256, 256)),
    (2048, 17408, 5120, (256, 256)), (4096, 17408, 5120, (256, 256)),
    (4096, 10240, 5120, (256, 160)), (4096, 5120, 8704, (256, 256))])
def test_plan_tile_shapes(lib, M, N, K, tile):
    k, v, s = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    assert lib.w4a8_plan(M, N, K, ctypes.byref(k), ctypes.byref(v), ctypes.byref(s)) == 0
    assert k.value == 2
    assert _native.variants(2)[v.value][2:] == tile


@pytest.mark.parametrize("M,N,K,stages,waves", [
    (17, 5120, 6144, 8, 4), (32, 17408, 5120, 8, 4), (64, 5120, 8704, 8, 4),
    (64, 10240, 5120, 5, 4), (64, 17408, 5120, 5, 8), (96, 5120, 8704, 8, 4),
    (96, 17408, 5120, 4, 8), (4096, 17408, 5120, 3, 8)])
def test_plan_pipeline_depth_and_waves(lib, M, N, K, stages, waves):
    """Narrow tiles run 8 stages deep (latency-bound at these M); large tiles 3-5, in 8 waves."""
    k, v, s = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    assert lib.w4a8_plan(M, N, K, ctypes.byref(k), ctypes.byref(v), ctypes.byref(s)) == 0
    c = _native.tile_config(v.value)
    assert (c["stages"], c["waves"]) == (stages, waves)


@pytest.mark.parametrize("M,N,K,cfg", [
    # shapes whose workgroups cover the chip: the fewest waves whose loads fit 160 registers
    # (4 per granule, 4 per activation k-tile at M <= 8, else 8), each wave owning a k-group
    (1, 10240, 5120, (3, 8, 5)), (8, 10240, 5120, (3, 8, 5)), (16, 10240, 5120, (3, 8, 5)),
    (1, 5120, 6144, (2, 12, 4)), (8, 5120, 6144, (2, 12, 4)), (16, 5120, 6144, (2, 8, 6)),
    (1, 5120, 8704, (2, 12, 6)), (8, 5120, 8704, (2, 12, 6)), (16, 5120, 8704, (2, 8, 9)),
    (1, 17408, 5120, (5, 4, 10)), (8, 17408, 5120, (5, 4, 10)), (16, 17408, 5120, (5, 4, 10)),
    # narrow shapes (fewer workgroups than half the CUs) or waves without a k-group: the fewest
    # granules on the busiest wave
    (8, 2048, 1024, (1, 4, 16)), (8, 1040, 512, (1, 4, 16)), (8, 48, 5120, (1, 4, 16))])
def test_plan_stream_variants(lib, M, N, K, cfg):
    """(n-tiles per workgroup, k-tiles per wave, waves) of the stream variant the plan takes."""
    k, v, s = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    assert lib.w4a8_plan(M, N, K, ctypes.byref(k), ctypes.byref(v), ctypes.byref(s)) == 0
    assert k.value == 3 and s.value == 1
    assert _native.variants(3)[v.value][:3] == cfg


def test_variant_tables(lib):
    sk = [(lib.w4a8_variant_count(1))]
    assert sk[0] > 0 and lib.w4a8_variant_count(2) > 0 and lib.w4a8_variant_count(9) == -1
    assert lib.w4a8_variant_count(3) > 0
    a = [ctypes.c_int() for _ in range(4)]
    assert lib.w4a8_variant_info(2, 0, *[ctypes.byref(x) for x in a]) == 0
    wm, wn, bm, bn = (x.value for x in a)
    assert bn == 32 * wn and bm % (32 * wm) == 0


def test_quant_and_repack_validate(lib):
    assert lib.w4a8_quant_per_token(None, 8, None, None, 4, 8, None) == 1
    assert lib.w4a8_quant_per_token(None, 8, None, None, 0, 8, None) == 0
    assert lib.w4a8_quant_per_token(4096, 4, 4096, 4096, 4, 8, None) == 1   # ldx < K
    assert lib.w4a8_repack(None, None, None, None, 16, 100, None) == 1


@pytest.mark.parametrize("K,msg", [(12, b"8-aligned"), (10248, b"<= 10240"), (0, b"8-aligned")])
def test_add_rms_quant_validates_before_launch(lib, K, msg):
    p = 4096
    assert lib.w4a8_add_rms_quant(p, p, p, p, p, p, 4, K, 1e-6, None, 0) == 1
    assert msg in lib.w4a8_last_error()


def test_producers_validate_before_launch(lib):
    p = 4096
    assert lib.w4a8_add_rms_quant(None, None, None, None, None, None, 0, 8, 1e-6, None, 0) == 0
    assert lib.w4a8_add_rms_quant(None, p, p, p, p, p, 4, 8, 1e-6, None, 0) == 1       # null y
    assert lib.w4a8_add_rms_quant(p + 2, p, p, p, p, p, 4, 8, 1e-6, None, 0) == 1      # misaligned
    assert lib.w4a8_silu_mul_quant(p, p, p, 4, 12, None, 0) == 1
    assert b"8-aligned" in lib.w4a8_last_error()
    assert lib.w4a8_silu_mul_quant(p, p, p, 4, 18440, None, 0) == 1
    assert lib.w4a8_silu_mul_quant(p, p + 4, p, 4, 16, None, 0) == 1                  # q misaligned
    assert lib.w4a8_silu_mul_quant(None, None, None, 0, 16, None, 0) == 0
    assert lib.w4a8_silu_mul(p, p, 4, 12, None) == 1
    assert b"w4a8_silu_mul: N must be 8-aligned" in lib.w4a8_last_error()
    assert lib.w4a8_silu_mul(p, p + 8, 4, 16, None) == 1                           # out misaligned
    assert lib.w4a8_silu_mul(p, None, 4, 16, None) == 1
    assert lib.w4a8_silu_mul(None, None, 0, 16, None) == 0
    assert lib.w4a8_gdn_norm_quant(p, p, 256, p, p, p, 4, 200, 1e-6, None, 0) == 1
    assert b"multiple of 128" in lib.w4a8_last_error()
    assert lib.w4a8_gdn_norm_quant(p, p, 100, p, p, p, 4, 128, 1e-6, None, 0) == 1     # stride < N
    assert lib.w4a8_gdn_norm_quant(p, p, 132, p, p, p, 4, 128, 1e-6, None, 0) == 1     # stride % 8
    assert b"stride" in lib.w4a8_last_error()
    assert lib.w4a8_gdn_norm_quant(p, p + 8, 256, p, p, p, 4, 128, 1e-6, None, 0) == 1  # z misaligned


def test_q_layout_is_validated(lib):
    p = 4096
    assert lib.w4a8_add_rms_quant(p, p, p, p, p, p, 4, 256, 1e-6, None, 2) == 1
    assert b"unknown q layout 2" in lib.w4a8_last_error()
    assert lib.w4a8_add_rms_quant(p, p, p, p, p, p, 4, 200, 1e-6, None, 1) == 1
    assert b"multiple of 128" in lib.w4a8_last_error()
    assert lib.w4a8_silu_mul_quant(p, p, p, 4, 8704 + 8, None, 1) == 1
    assert b"fragment-tiled" in lib.w4a8_last_error()
    assert lib.w4a8_gdn_norm_quant(p, p, 256, p, p, p, 4, 128, 1e-6, None, -1) == 1
    assert b"unknown q layout" in lib.w4a8_last_error()
    # M = 0 with a valid tiled layout is a no-op
    assert lib.w4a8_silu_mul_quant(None, None, None, 0, 8704, None, 1) == 0


def test_tiled_gemm_validates_before_launch(lib):
    p = 4096
    assert lib.w4a8_gemm_at(p, p, p, p, p, 64, 256, 5120 + 32, None) == 1
    assert b"K % 128" in lib.w4a8_last_error()
    assert lib.w4a8_gemm_at(None, p, p, p, p, 64, 256, 5120, None) == 1          # null a
    assert lib.w4a8_gemm_at(None, None, None, None, None, 0, 256, 5120, None) == 0
    # fragment-tiled activations go to the tile and ring kernels only
    assert lib.w4a8_gemm_planned(p, p, p, p, p, 8, 256, 512, _native.KERNEL_TILE_AT, 99, 1,
                                 None) == 1
    assert b"tile variant 99 out of range" in lib.w4a8_last_error()
    assert lib.w4a8_variant_count(_native.KERNEL_TILE_AT) == \
        lib.w4a8_variant_count(_native.KERNEL_TILE)
    assert lib.w4a8_gemm_planned(p, p, p, p, p, 32, 256, 5120 + 32, _native.KERNEL_RING_AT, 0, 1,
                                 None) == 1
    assert b"K % 128" in lib.w4a8_last_error()
    assert lib.w4a8_gemm_planned(p, p, p, p, p, 32, 256, 512, _native.KERNEL_RING_AT, 99, 1,
                                 None) == 1
    assert b"ring variant 99 out of range" in lib.w4a8_last_error()
    assert lib.w4a8_variant_count(_native.KERNEL_RING_AT) == \
        lib.w4a8_variant_count(_native.KERNEL_RING)


def test_tile_k_split_validates_before_launch(lib):
    """A forced tile plan with split_k > 1 splits K over workgroup rows: it needs a variant with a
    K-split form (the 4-wave tiles up to 64 tokens tall), N % 16 == 0, at most one split per
    k-group, and registered scratch for the fp32 partials."""
    p = 1 << 20
    big = next(v for v, c in enumerate(_native.variants(_native.KERNEL_TILE)) if c[2] == 256)
    assert lib.w4a8_gemm_planned(p, p, p, p, p, 32, 1024, 8704, _native.KERNEL_TILE, big, 3,
                                 None) == 1
    assert b"no K-split form" in lib.w4a8_last_error()
    assert lib.w4a8_gemm_planned(p, p, p, p, p, 32, 1000, 8704, _native.KERNEL_TILE, 0, 3,
                                 None) == 1
    assert b"N % 16 == 0" in lib.w4a8_last_error()
    assert lib.w4a8_gemm_planned(p, p, p, p, p, 32, 1024, 1024, _native.KERNEL_TILE, 0, 3,
                                 None) == 1
    assert b"one split per k-group (2)" in lib.w4a8_last_error()
    assert lib.w4a8_gemm_planned(p, p, p, p, p, 32, 1024, 8704, _native.KERNEL_TILE, 0, 3,
                                 None) == 2
    assert b"needs 393216 B of partials" in lib.w4a8_last_error()


@pytest.mark.parametrize("M,K,want", [(0, 128, 0), (1, 128, 2048), (16, 5120, 16 * 5120),
                                      (17, 8704, 32 * 8704), (4096, 5120, 4096 * 5120)])
def test_tiled_bytes(lib, M, K, want):
    n = ctypes.c_size_t()
    assert lib.w4a8_tiled_bytes(M, K, ctypes.byref(n)) == 0
    assert n.value == want


def test_tiled_bytes_refuses_ragged_k(lib):
    n = ctypes.c_size_t()
    assert lib.w4a8_tiled_bytes(4, 96, ctypes.byref(n)) == 1
    assert lib.w4a8_tiled_bytes(4, 128, None) == 1


def test_read_probe_validates_before_launch(lib):
    p = 4096
    assert lib.w4a8_read_probe(None, 1024, p, None) == 1
    assert lib.w4a8_read_probe(p, 0, p, None) == 1
    assert lib.w4a8_read_probe(p + 4, 1024, p, None) == 1                         # misaligned
    assert lib.w4a8_read_probe(p, 1 << 31, p, None) == 1
    assert b"w4a8_read_probe" in lib.w4a8_last_error()


def test_read_probe_shape_validates_before_launch(lib):
    """The launch-shape sweep of the read probe: every variant describes itself, and a grid whose
    workgroups the variant cannot cover, or that leaves a workgroup without bytes, is refused."""
    n = lib.w4a8_read_probe_variants()
    assert n >= 16
    p = [ctypes.c_int() for _ in range(4)]
    for v in range(n):
        assert lib.w4a8_read_probe_variant_info(v, *[ctypes.byref(x) for x in p]) == 0
        waves, units, window, nt = (x.value for x in p)
        assert 1 <= waves <= 16 and 1 <= window <= units and nt in (0, 1)
    assert lib.w4a8_read_probe_variant_info(n, *[ctypes.byref(x) for x in p]) == 1
    b = 4096
    nbytes = 47_669_280
    assert lib.w4a8_read_probe_shape(None, nbytes, b, 218, 1, None) == 1
    assert lib.w4a8_read_probe_shape(b + 4, nbytes, b, 218, 1, None) == 1          # misaligned
    assert lib.w4a8_read_probe_shape(b, 1 << 31, b, 218, 1, None) == 1
    assert lib.w4a8_read_probe_shape(b, nbytes, b, 100, 1, None) == 1       # 10 x 22 KiB < share
    assert lib.w4a8_read_probe_shape(b, nbytes, b, 1012, 12, None) == 1    # last workgroup empty
    assert lib.w4a8_read_probe_shape(b, nbytes, b, 218, n, None) == 1
    assert b"w4a8_read_probe_shape" in lib.w4a8_last_error()


def test_stream_load_probe_validates_before_launch(lib):
    """The streaming GEMM's loads alone: only shapes the plan sends to the streaming kernel at
    M <= 8, the three load sets, and the GEMM's operand checks."""
    p = 4096
    assert lib.w4a8_stream_load_probe(p, p, p, p, 0, 17408, 5120, 7, p, None) == 1
    assert lib.w4a8_stream_load_probe(p, p, p, p, 9, 17408, 5120, 7, p, None) == 1
    for parts in (0, 2, 4, 5, 8):
        assert lib.w4a8_stream_load_probe(p, p, p, p, 8, 17408, 5120, parts, p, None) == 1
    assert b"parts" in lib.w4a8_last_error()
    assert lib.w4a8_stream_load_probe(p, p, p, p, 8, 17408, 5000, 7, p, None) == 1
    assert lib.w4a8_stream_load_probe(None, p, p, p, 8, 17408, 5120, 7, p, None) == 1
    assert lib.w4a8_stream_load_probe(p, p, p, p, 8, 17408, 5120, 7, None, None) == 1
    assert lib.w4a8_stream_load_probe(p + 4, p, p, p, 8, 17408, 5120, 7, p, None) == 1
    assert lib.w4a8_stream_load_probe(p, p, p, p, 8, 33, 640, 7, p, None) == 1   # skinny plan
    assert b"not the streaming GEMM" in lib.w4a8_last_error()


def test_workspace_bytes_covers_the_band_split_in_4_mib(lib):
    """The scratch the plugin registers, sized by the library's own plan: the skinny kernel's
    split-K partials for small-N shapes at M <= 16, SiLU-mul's split-row maxima, and the band's
    three-way K split of the tile kernel (fp32 partials of 3 x M x N, M <= 48), which fires only
    where the unsplit grid leaves half the CUs idle (N <= 85 x 64 = 5440 on 256 CUs): 3.1 MB in
    all, within the allocation-free entry point's 4 MiB (the reference registered 37.7 MB,
    sly/mxfp4/radiance_mxfp4.py:1064-1070)."""
    part, cnt = _native.workspace_bytes(64, 36864)
    assert part == 3 * 48 * 5440 * 4 and 0 < cnt <= 4096
    assert part <= 4 << 20
    # down (N = 5120) at M = 48 fits; without the band (M <= 16) it stays under 1 MiB
    assert _native.workspace_bytes(64, 5120)[0] == 3 * 48 * 5120 * 4
    assert 9216 <= _native.workspace_bytes(16, 36864)[0] < 1 << 20
    # monotone in the limits, and never below SiLU-mul's own need (64 rows x 36 chunks x 4 B)
    p2, c2 = _native.workspace_bytes(64, 65536)
    assert p2 >= part and c2 >= cnt
    assert _native.workspace_bytes(1, 16)[0] >= 36 * 4
    for bad in ((0, 16), (1, 0), (1, (1 << 22) + 1)):
        with pytest.raises(RuntimeError):
            _native.workspace_bytes(*bad)
