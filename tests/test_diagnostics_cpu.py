"""The op's in-situ diagnostics (vllm_sly_radiance_amd/diagnostics.py), on the CPU: the torch
unrepack inverts the oracle's repack, the exact check's reference equals the oracle's fp32 GEMM,
and the CHECKALL / MHIST reporting counts and prints what the reference's does
(sly/mxfp4/radiance_mxfp4.py:755-785)."""
import numpy as np
import pytest
import torch

from oracle import mxfp4_oracle as O
from vllm_sly_radiance_amd import diagnostics as D
from vllm_sly_radiance_amd import synthetic


def _layer(N, K, seed):
    w, ws = synthetic.weights(N, K, seed=seed)
    wq, sq = O.repack(w, ws)
    return w, ws, torch.from_numpy(wq.reshape(-1)), torch.from_numpy(sq.reshape(-1).view(np.uint8))


@pytest.mark.parametrize("N,K", [(32, 512), (48, 1024), (40, 96), (17, 544)])
def test_unrepack_inverts_the_repack(N, K):
    w, ws, wq, sq = _layer(N, K, N + K)
    gw, gs = D.unrepack(wq, sq, N, K)
    assert np.array_equal(gw.numpy(), w) and np.array_equal(gs.numpy(), ws)


@pytest.mark.parametrize("M,N,K", [(3, 48, 512), (8, 40, 96)])
def test_exact_linear_is_the_oracle_gemm(M, N, K):
    w, ws, wq, sq = _layer(N, K, 7 * N + K)
    q, s = O.quant_per_token(synthetic.activations(M, K, seed=M + N))
    got = D.exact_linear(torch.from_numpy(q), torch.from_numpy(s), wq, sq, N, K, chunk=16).numpy()
    ref = O.gemm_ref_f32(q, s, w, ws)
    exact = O.gemm_exact_f64(q, s, w, ws)
    bound = 1e-5 * O.gemm_abs_terms(q, s, w, ws) + 1e-30
    assert np.all(np.abs(got - exact) <= bound) and np.all(np.abs(ref - exact) <= bound)


def _case(M=4, N=32, K=512):
    w, ws, wq, sq = _layer(N, K, 3)
    q, s = O.quant_per_token(synthetic.activations(M, K, seed=11))
    y = O.gemm_ref_f32(q, s, w, ws)
    out = torch.from_numpy(y).to(torch.bfloat16)
    return torch.from_numpy(q), torch.from_numpy(s), wq, sq, out, N, K


@pytest.fixture
def diag(monkeypatch):
    monkeypatch.setattr(D, "CHECK_ALL", {(32, 512)})
    monkeypatch.setattr(D, "CHECK_MAX_M", 128)
    monkeypatch.setattr(D, "MHIST", True)
    monkeypatch.setattr(D, "_seen", set())
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    return D


def test_checkall_reports_ok_then_wrong(diag, capsys):
    q, s, wq, sq, out, N, K = _case()
    stats = {}
    diag.after_call(stats, q, s, wq, sq, out, N, K)
    err = capsys.readouterr().err
    assert "[radiance.mxfp4.mhist] N=32 K=512 M=4 plan=" in err
    assert "[radiance.mxfp4.all] ok N=32 K=512 M=4 call#1" in err
    assert stats["checked"] == 1 and stats.get("wrong", 0) == 0
    diag.after_call(stats, q, s, wq, sq, out, N, K)          # mhist once; no second ok line
    assert capsys.readouterr().err == ""
    bad = out.clone()
    bad[:, :16] = -bad[:, :16]                                # a sign error on half the columns
    diag.after_call(stats, q, s, wq, sq, bad, N, K)
    assert "**WRONG** call#3 N=32 K=512 M=4" in capsys.readouterr().err
    assert stats["wrong"] == 1
    nan = out.clone()
    nan[0, 0] = float("nan")
    diag.after_call(stats, lambda: (q, s), None, wq, sq, nan, N, K)   # NaN counts as wrong
    assert stats["wrong"] == 2 and stats["checked"] == 4


def test_checkall_skips_other_shapes_large_m_and_capture(diag, capsys, monkeypatch):
    q, s, wq, sq, out, N, K = _case()
    stats = {}
    monkeypatch.setattr(D, "CHECK_ALL", {(64, 512)})
    diag.after_call(stats, q, s, wq, sq, out, N, K)
    monkeypatch.setattr(D, "CHECK_ALL", {(32, 512)})
    monkeypatch.setattr(D, "CHECK_MAX_M", 2)
    diag.after_call(stats, q, s, wq, sq, out, N, K)
    monkeypatch.setattr(D, "CHECK_MAX_M", 128)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    diag.after_call(stats, q, s, wq, sq, out, N, K)
    assert "checked" not in stats
    assert capsys.readouterr().err.count("[radiance.mxfp4.mhist]") == 1


def test_parse_shapes_and_report_stats(capsys, monkeypatch):
    assert D.parse_shapes("") is None
    assert D.parse_shapes("17408:5120, 5120:8704,") == {(17408, 5120), (5120, 8704)}
    monkeypatch.setattr(D, "_reported", [False])
    D.report_stats({"fast": 3, "refused": 1})
    D.report_stats({"fast": 9, "refused": 9})
    err = capsys.readouterr().err
    assert err.count("[radiance.mxfp4] linear layers: 3/4 on the gfx950 W4A8 kernels, 1 refused") == 1


def test_sanitize_zeroes_non_finite_inputs(monkeypatch):
    x = torch.tensor([[1.0, float("nan"), float("inf"), -float("inf"), -2.5]], dtype=torch.bfloat16)
    monkeypatch.setattr(D, "SANITIZE_X", False)
    assert D.sanitize(x) is x
    monkeypatch.setattr(D, "SANITIZE_X", True)
    y = D.sanitize(x)
    assert y.dtype == torch.bfloat16 and y.tolist() == [[1.0, 0.0, 0.0, 0.0, -2.5]]
    assert torch.isnan(x[0, 1])                              # the input itself is left alone


def test_health_report_once_per_shape_and_capped(diag, capsys, monkeypatch):
    q, s, wq, sq, out, N, K = _case()
    monkeypatch.setattr(D, "CHECK_X", True)
    monkeypatch.setattr(D, "CHECK_ALL", None)
    monkeypatch.setattr(D, "MHIST", False)
    x = torch.ones((out.shape[0], K), dtype=torch.bfloat16)
    x[0, 0] = float("nan")
    D.after_call({}, q, s, wq, sq, out, N, K, x=x)
    D.after_call({}, q, s, wq, sq, out, N, K, x=x)
    err = capsys.readouterr().err
    assert err.count("[radiance.mxfp4.x] N=32 K=512 M=4 ") == 1 and "x_nonfin=1 " in err
    assert "out_nonfin=0" in err
    monkeypatch.setattr(D, "CHECK_X_MAX", 1)
    D.after_call({}, q, s, wq, sq, out[:2], N, K)               # a new shape past the cap
    assert capsys.readouterr().err == ""


def test_debug_reports_each_shape_once(diag, capsys, monkeypatch):
    """RADIANCE_MXFP4_DEBUG: one exact comparison per (N, K, M), ok or wrong, up to DEBUG_MAX
    shapes, not above M = 128 and not under capture; no tally is kept."""
    monkeypatch.setattr(D, "CHECK_ALL", None)
    monkeypatch.setattr(D, "MHIST", False)
    monkeypatch.setattr(D, "DEBUG", True)
    q, s, wq, sq, out, N, K = _case()
    stats = {}
    D.after_call(stats, q, s, wq, sq, out, N, K)
    err = capsys.readouterr().err
    assert "[radiance.mxfp4.exact] N=32 K=512 M=4 rel_vs_fp32=" in err and err.rstrip().endswith("ok")
    D.after_call(stats, q, s, wq, sq, out, N, K)
    assert capsys.readouterr().err == ""                      # once per shape
    q2, s2, _, _, out2, _, _ = _case(M=2)
    bad = out2.clone()
    bad[:, :16] = -bad[:, :16]
    D.after_call(stats, q2, s2, wq, sq, bad, N, K)
    assert "M=2" in (e := capsys.readouterr().err) and "**WRONG**" in e
    assert stats == {}
    monkeypatch.setattr(D, "DEBUG_MAX", 2)                    # two shapes seen: no more
    q3, s3, _, _, out3, _, _ = _case(M=3)
    D.after_call(stats, q3, s3, wq, sq, out3, N, K)
    assert capsys.readouterr().err == ""


def test_padded_and_cloned_output(monkeypatch):
    """RADIANCE_MXFP4_PADOUT=n: the output is an [M, N] view n elements into a slab with n spare
    elements on each side. RADIANCE_MXFP4_CLONE=1: the op returns a copy."""
    monkeypatch.setattr(D, "PAD_OUT", 0)
    o = D.new_out(3, 40, "cpu")
    assert o.shape == (3, 40) and o.dtype == torch.bfloat16 and o.untyped_storage().nbytes() == 240
    monkeypatch.setattr(D, "PAD_OUT", 5)
    o = D.new_out(3, 40, "cpu")
    assert o.shape == (3, 40) and o.is_contiguous() and o.storage_offset() == 5
    assert o.untyped_storage().nbytes() == 2 * (120 + 10)
    monkeypatch.setattr(D, "CLONE_OUT", False)
    assert D.returned(o) is o
    monkeypatch.setattr(D, "CLONE_OUT", True)
    o.fill_(1.5)
    c = D.returned(o)
    assert c.data_ptr() != o.data_ptr() and torch.equal(c, o)
