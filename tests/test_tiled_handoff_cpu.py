"""Host logic of the fragment-tiled handoff (radiance_mxfp4.TiledHandoff, a_tiled_wanted,
alloc_tiled_q), on CPU tensors: what a producer records, what mxfp4_linear_pq accepts, and what it
refuses (other shapes, row-major storage at a recorded address, records aged out). Mirrors the
behaviour of the reference's data_ptr table (sly/mxfp4/radiance_mxfp4.py:54-80)."""
import pytest
import torch

from vllm_sly_radiance_amd import radiance_mxfp4 as R


def test_alloc_is_a_row_view_over_whole_blocks_plus_tail():
    q = R.alloc_tiled_q(17, 256, "cpu")
    assert tuple(q.shape) == (17, 256) and q.is_contiguous()
    assert q.dtype == torch.float8_e4m3fn
    assert q.untyped_storage().nbytes() == 32 * 256 + 128


def test_mark_then_claim_repeatedly():
    h = R.TiledHandoff()
    q = R.alloc_tiled_q(130, 512, "cpu")
    assert not h.claim(q, 130, 512)
    h.mark(q, 130, 512)
    assert h.claim(q, 130, 512) and h.claim(q, 130, 512)     # several consumers


def test_shape_mismatch_drops_the_record():
    h = R.TiledHandoff()
    q = R.alloc_tiled_q(130, 512, "cpu")
    h.mark(q, 130, 512)
    assert not h.claim(q, 130, 256)
    assert not h.claim(q, 130, 512)


def test_row_major_storage_is_never_taken_for_tiled():
    h = R.TiledHandoff()
    q = torch.empty((128, 512), dtype=torch.float8_e4m3fn)
    h.mark(q, 128, 512)                 # a caller recording a row-major tensor by mistake
    assert not h.claim(q, 128, 512)


def test_views_into_tiled_storage():
    # whole 16-token blocks are contiguous, so dropping leading blocks leaves a tiled tensor of
    # the remaining tokens; any other row offset is not one
    h = R.TiledHandoff()
    q = R.alloc_tiled_q(64, 256, "cpu")
    whole, ragged = q[16:], q[5:]
    h.mark(whole, 48, 256)
    h.mark(ragged, 59, 256)
    assert h.claim(whole, 48, 256)
    assert not h.claim(ragged, 59, 256)


def test_records_age_out():
    h = R.TiledHandoff(keep=4)
    qs = [R.alloc_tiled_q(80, 128, "cpu") for _ in range(6)]
    for q in qs:
        h.mark(q, 80, 128)
    assert [h.claim(q, 80, 128) for q in qs] == [False, False, True, True, True, True]


def test_remark_moves_a_record_to_the_newest():
    h = R.TiledHandoff(keep=2)
    a, b, c = (R.alloc_tiled_q(80, 128, "cpu") for _ in range(3))
    h.mark(a, 80, 128)
    h.mark(b, 80, 128)
    h.mark(a, 80, 128)
    h.mark(c, 80, 128)
    assert h.claim(a, 80, 128) and not h.claim(b, 80, 128)


def test_wanted_threshold(monkeypatch):
    monkeypatch.setattr(R, "A_TILED_MIN_M", 0)
    assert not R.a_tiled_wanted(4096)
    monkeypatch.setattr(R, "A_TILED_MIN_M", 1024)
    assert not R.a_tiled_wanted(1023) and R.a_tiled_wanted(1024)


def test_threshold_inside_the_decode_band_is_refused():
    import subprocess
    import sys
    code = "import vllm_sly_radiance_amd.radiance_mxfp4"
    env = dict(__import__("os").environ, RADIANCE_MXFP4_A_TILED_MIN_M="64")
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                       cwd=__import__("os").path.dirname(__import__("os").path.dirname(
                           __import__("os").path.abspath(__file__))))
    assert r.returncode != 0 and "must exceed 64" in r.stderr


@pytest.mark.parametrize("M,K,tiled", [(4096, 5120, True), (4096, 200, False), (64, 5120, False)])
def test_producers_ask_for_tiles_only_past_the_threshold(monkeypatch, M, K, tiled):
    from vllm_sly_radiance_amd import radiance_fused_norm as FN
    monkeypatch.setattr(R, "A_TILED_MIN_M", 65)
    assert FN._tiled(M, K) == tiled
