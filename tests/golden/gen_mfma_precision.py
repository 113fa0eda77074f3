#!/usr/bin/env python3
"""Measure the accumulation precision of the gfx950 scaled MFMA the GEMMs issue (16x16x128, fp4
e2m1 A x fp8 e4m3 B) on an MI355X and write the raw tiles as a golden fixture.

    python tests/golden/gen_mfma_precision.py [out.npz]   (needs the GPU and the built library)

Tiles go through the library's w4a8_mfma_tile diagnostic. Families (operands + hardware result):
  narrow        fp8 values with one exponent (1.0 .. 1.875, random sign) x random fp4, unit scales:
                every product sum fits a narrow window, so the result is the exact sum
  big_small     every product 2^-6 except one big product per 16-element run of k, the big one
                stepping through fp8 magnitudes: shows which small products the hardware drops
  block_spread  unit products, the first 32-block scaled by 2^s, s = 0..39: shows the precision
                with which 8-product group sums are combined
  random        random codes, random scales in [118, 136] on both operands
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)


def tiles(a, b, sa, sb):
    import torch
    from vllm_sly_radiance_amd import _native
    T = a.shape[0]
    ad = torch.from_numpy(np.ascontiguousarray(a, np.uint8).view(np.int32)).cuda()
    bd = torch.from_numpy(np.ascontiguousarray(b, np.uint8).view(np.int32)).cuda()
    sad = torch.from_numpy(np.ascontiguousarray(sa, np.int32)).cuda()
    sbd = torch.from_numpy(np.ascontiguousarray(sb, np.int32)).cuda()
    d = torch.empty((T, 64, 4), dtype=torch.float32, device="cuda")
    assert ad.shape == (T, 64, 4) and bd.shape == (T, 64, 8) and sad.shape == sbd.shape == (T, 64)
    _native.mfma_tile(ad.data_ptr(), bd.data_ptr(), sad.data_ptr(), sbd.data_ptr(), d.data_ptr(), T,
                      torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return d.cpu().numpy()


def families(rng):
    fam = {}
    unit = lambda T: np.full((T, 64), 127, np.int32)
    T = 64
    a = rng.integers(0, 256, (T, 64, 16), dtype=np.uint8)
    b = ((rng.integers(0, 2, (T, 64, 32)) << 7) | (7 << 3)
         | rng.integers(0, 8, (T, 64, 32))).astype(np.uint8)
    fam["narrow"] = (a, b, unit(T), unit(T))
    T = 60
    a = np.full((T, 64, 16), 0x22, np.uint8)                        # every fp4 element 1.0
    b = np.full((T, 64, 32), 0x08, np.uint8)                        # every fp8 element 2^-6
    for t in range(T):
        b[t, :, 0] = (min(15, 1 + t // 4) << 3) | (t % 8)           # byte 0 of every lane: big
    fam["big_small"] = (a, b, unit(T), unit(T))
    T = 40
    a = np.full((T, 64, 16), 0x22, np.uint8)
    b = np.full((T, 64, 32), 0x38, np.uint8)
    sa = unit(T).copy()
    sa[:, :16] += np.arange(T)[:, None]                             # block 0 of every row
    fam["block_spread"] = (a, b, sa, unit(T))
    T = 64
    a = rng.integers(0, 256, (T, 64, 16), dtype=np.uint8)
    b = rng.integers(0, 256, (T, 64, 32), dtype=np.uint8)
    b = np.where((b & 0x7F) == 0x7F, 0x38, b).astype(np.uint8)
    fam["random"] = (a, b, rng.integers(118, 137, (T, 64)).astype(np.int32),
                     rng.integers(118, 137, (T, 64)).astype(np.int32))
    return fam


def main():
    out = sys.argv[1] if len(sys.argv) > 1 else os.path.join(
        ROOT, "tests", "golden", "mfma_16x16x128_f4f8_precision.npz")
    import torch
    res = {"device": np.array(torch.cuda.get_device_properties(0).gcnArchName)}
    for name, (a, b, sa, sb) in families(np.random.default_rng(2026)).items():
        res.update({f"{name}_a": a, f"{name}_b": b, f"{name}_sa": sa, f"{name}_sb": sb,
                    f"{name}_d": tiles(a, b, sa, sb)})
    np.savez_compressed(out, **res)
    print(f"wrote {out}")


if __name__ == "__main__":
    main()
