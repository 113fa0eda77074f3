"""The allocation-free GEMM entry point (w4a8_gemm_noalloc) against w4a8_gemm_planned.

w4a8_gemm_noalloc keeps its split-K partials and counters in the library's static device array
instead of registered scratch; with the same plan it runs the same kernels, so its outputs must
equal w4a8_gemm_planned's bit for bit (and so meet the GEMM tolerance against the oracle). Checked
on two calls in a row, the second with a smaller input, for split-K plans (the static scratch in
use) and a plan without a split; a forced plan whose partials exceed the static array is refused
before anything launches; torch's caching allocator records no allocation during a call."""
import numpy as np
import pytest
import torch

from oracle import mxfp4_oracle as O
from tests._check import assert_gemm_close, host_u16, stream, to_dev
from vllm_sly_radiance_amd import _native, synthetic

pytestmark = pytest.mark.gpu

SKINNY = _native.KERNEL_SKINNY


@pytest.fixture(scope="module")
def registered(gpu_lib):
    """Registered scratch for the reference side (w4a8_gemm_planned): room for every plan these
    tests force. The plugin's own registration is put back afterwards."""
    from vllm_sly_radiance_amd import radiance_mxfp4 as R
    R.ensure_scratch("cuda")
    part = torch.empty(16 << 20, dtype=torch.uint8, device="cuda")
    cnt = torch.zeros(4096, dtype=torch.int32, device="cuda")
    _native.set_scratch(part.data_ptr(), part.numel(), cnt.data_ptr(), cnt.numel() * 4)
    yield part, cnt
    torch.cuda.synchronize()
    p, c = R._scratch
    _native.set_scratch(p.data_ptr(), p.numel() * 4, c.data_ptr(), c.numel() * 4)


def operands(M, N, K, seed):
    x = synthetic.activations(M, K, seed=seed)
    w, ws = synthetic.weights(N, K, seed=seed + 1)
    q, s = O.quant_per_token(x)
    wb, sb = _native.packed_bytes(N, K)
    wq = torch.empty(wb, dtype=torch.uint8, device="cuda")
    sq = torch.empty(sb, dtype=torch.uint8, device="cuda")
    wd, sd = to_dev(w), to_dev(ws)
    _native.repack(wd.data_ptr(), sd.data_ptr(), wq.data_ptr(), sq.data_ptr(), N, K, stream())
    return dict(q=q, s=s, w=w, ws=ws, qd=to_dev(q), sd=to_dev(s), wq=wq, sq=sq, M=M, N=N, K=K)


def run(fn, op, kernel=_native.KERNEL_AUTO, variant=-1, split=0):
    """fn on op's operands into a fresh output; returns (output, torch allocations the call made:
    the count of allocation events of the caching allocator across the call alone)."""
    M, N, K = op["M"], op["N"], op["K"]
    out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    count = lambda: torch.cuda.memory_stats().get("allocation.all.allocated", 0)
    before = count()
    fn(op["qd"].data_ptr(), op["sd"].data_ptr(), op["wq"].data_ptr(), op["sq"].data_ptr(),
       out.data_ptr(), M, N, K, stream(), kernel, variant, split)
    return out, count() - before


# (M, N, K) pairs: first call, then a smaller one. 65 and 33 n-tiles plan split-K on the skinny
# kernel; N = 2048, K = 5120 plans the streaming kernel (no scratch); down-shaped K = 8704 at
# M = 32 and 17 plans the tile kernel with K split three ways (fp32 partials in the scratch).
CASES = [((8, 1040, 2560), (3, 528, 1024)), ((16, 2048, 5120), (5, 1040, 2560)),
         ((32, 5120, 8704), (17, 1024, 8704))]


@pytest.mark.parametrize("first,second", CASES)
def test_noalloc_equals_planned_twice(registered, first, second):
    for shape, seed in ((first, 1), (second, 2)):
        op = operands(*shape, seed=seed)
        plan = _native.plan(*shape)
        print(f"[noalloc] M,N,K={shape} plan {plan}", flush=True)
        if shape[2] == 8704:                     # the band's tile K split is what runs here
            assert plan[0] == _native.KERNEL_TILE and plan[2] == 3, plan
        got, allocs = run(_native.gemm_noalloc, op)
        assert allocs == 0
        want, _ = run(_native.gemm, op)
        torch.cuda.synchronize()
        a, b = host_u16(got), host_u16(want)
        bad = np.argwhere(a != b)
        assert bad.size == 0, f"{shape}: {len(bad)} outputs differ from w4a8_gemm, first {bad[:3]}"
        assert_gemm_close(a, op["q"], op["s"], op["w"], op["ws"], f"noalloc {shape} plan {plan}")


def test_noalloc_split_plan_uses_the_static_scratch(registered):
    """A forced split-K plan (16 splits of 65 n-tiles) through both entry points, twice in a row
    with different inputs: the static counters reset themselves between calls."""
    v = [i for i, c in enumerate(_native.variants(SKINNY)) if c[:3] == (1, 1, 16)][0]
    for seed in (3, 4):
        op = operands(7, 1040, 2560, seed=seed)
        got, allocs = run(_native.gemm_noalloc, op, SKINNY, v, 16)
        want, _ = run(_native.gemm, op, SKINNY, v, 16)
        assert allocs == 0
        got, want = host_u16(got), host_u16(want)
        torch.cuda.synchronize()
        assert np.array_equal(got, want)
        assert_gemm_close(got, op["q"], op["s"], op["w"], op["ws"],
                          f"noalloc forced split seed {seed}")


def test_noalloc_refuses_a_split_beyond_its_static_scratch(registered):
    """16 splits over 2304 n-tiles need 37.7 MB of partials: refused before any launch."""
    v = [i for i, c in enumerate(_native.variants(SKINNY)) if c[:3] == (1, 1, 16)][0]
    p = 1 << 20
    rc = _native.lib().w4a8_gemm_noalloc(p, p, p, p, p, 8, 36864, 5120, SKINNY, v, 16, None)
    assert rc == 2
    assert b"static scratch" in _native.lib().w4a8_last_error()


def test_noalloc_refuses_a_tile_split_beyond_its_static_scratch(registered):
    """A forced three-way K split of the 64 x 64 band tile at M = 48, N = 16384 needs 9.4 MB of
    partials: refused before any launch."""
    v = [i for i, c in enumerate(_native.variants(_native.KERNEL_TILE))
         if c[2:] == (64, 64) and _native.tile_config(i)["stages"] == 5][0]
    p = 1 << 20
    rc = _native.lib().w4a8_gemm_noalloc(p, p, p, p, p, 48, 16384, 8704, _native.KERNEL_TILE, v,
                                         3, None)
    assert rc == 2
    assert b"static scratch" in _native.lib().w4a8_last_error()


def test_noalloc_under_graph_capture(registered):
    """w4a8_gemm_noalloc captured into a HIP graph on a split plan (down 5120 x 8704 at M = 24: the
    band tile with K in three, partials in the static array), replayed three times with eager
    split calls of another shape between the replays (they overwrite the same static partials):
    every replay equals the eager call bit for bit. The capture itself allocates nothing through
    the entry point (the set-up call ran eagerly in the tests above)."""
    op = operands(24, 5120, 8704, seed=5)
    other = operands(17, 5120, 8704, seed=6)
    plan = _native.plan(24, 5120, 8704)
    assert plan[0] == _native.KERNEL_TILE and plan[2] == 3, plan
    eager, _ = run(_native.gemm_noalloc, op)
    other_eager, _ = run(_native.gemm_noalloc, other)
    torch.cuda.synchronize()
    want, want_other = host_u16(eager), host_u16(other_eager)
    out = torch.full((24, 5120), float("nan"), dtype=torch.bfloat16, device="cuda")
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        _native.gemm_noalloc(op["qd"].data_ptr(), op["sd"].data_ptr(), op["wq"].data_ptr(),
                             op["sq"].data_ptr(), out.data_ptr(), 24, 5120, 8704,
                             side.cuda_stream)
    for r in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        print(f"[noalloc] graph replay {r}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host_u16(out), want), f"replay {r}"
        got_other, _ = run(_native.gemm_noalloc, other)
        torch.cuda.synchronize()
        assert np.array_equal(host_u16(got_other), want_other), f"eager call after replay {r}"
    del graph
