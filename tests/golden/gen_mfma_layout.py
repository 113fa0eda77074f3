#!/usr/bin/env python3
"""Measure the lane layout of the gfx950 scaled MFMA the GEMMs issue (16x16x128, fp4 e2m1 A x fp8
e4m3 B, per-lane e8m0 scales) on an MI355X and write it as a label-free golden fixture.

    python tests/golden/gen_mfma_layout.py [out.npz]     (needs the GPU and the built library)

Every tile goes through the library's w4a8_mfma_tile diagnostic. Experiments (one tile each):
  R   one A nibble = 1.0, every B byte = 1.0      -> the D positions an A lane's row lights
  C   one B byte = 1.0, every A nibble = 1.0      -> the D positions a B lane's column lights
  K   one B byte = 1.0, A nibble (lane, j) = bit b of (32 lane + j), b = 0..10
                                                  -> which A element each B element meets, per row
  SA  one B byte = 1.0, A all 1.0, A-lane scale = 127 + bit b of the lane, b = 0..5
  SB  same with the B-lane scales                 -> which scale lanes apply to each product
Output arrays (all integers; D positions are lane * 4 + register):
  a_row_pos [64, 16]      sorted D positions lit by A lane la
  b_col_pos [64, 16]      sorted D positions lit by B lane lb
  meet      [64, 32, 16]  for B byte (lb, jb) and the i-th D position of its column: the A element
                          (32 * lane + nibble) it is multiplied with
  sa_lane   [64, 32, 16]  the A-scale lane applied to that product
  sb_lane   [64, 32, 16]  the B-scale lane applied to that product
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

ONE_FP4, ONE_FP8 = 2, 0x38
P = 64 * 32


def fp4_bytes(nib):
    return (nib[..., 0::2] | (nib[..., 1::2] << 4)).astype(np.uint8)


def tiles(a_nib, b, sa, sb):
    import torch
    from vllm_sly_radiance_amd import _native
    T = a_nib.shape[0]
    a = torch.from_numpy(np.ascontiguousarray(fp4_bytes(a_nib)).view(np.int32)).cuda()
    bd = torch.from_numpy(np.ascontiguousarray(b, np.uint8).view(np.int32)).cuda()
    sad = torch.from_numpy(np.ascontiguousarray(sa, np.int32)).cuda()
    sbd = torch.from_numpy(np.ascontiguousarray(sb, np.int32)).cuda()
    d = torch.empty((T, 64, 4), dtype=torch.float32, device="cuda")
    assert a.shape == (T, 64, 4) and bd.shape == (T, 64, 8) and sad.shape == sbd.shape == (T, 64)
    _native.mfma_tile(a.data_ptr(), bd.data_ptr(), sad.data_ptr(), sbd.data_ptr(), d.data_ptr(), T,
                      torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return d.cpu().numpy().reshape(T, 256)


def measure():
    unit = np.full((P, 64), 127, np.int32)
    one_b = np.zeros((P, 64, 32), np.uint8)
    one_b[np.arange(P), np.arange(P) // 32, np.arange(P) % 32] = ONE_FP8
    one_a = np.zeros((P, 64, 32), np.uint8)
    one_a[np.arange(P), np.arange(P) // 32, np.arange(P) % 32] = ONE_FP4
    all_a = np.full((P, 64, 32), ONE_FP4, np.uint8)
    dR = tiles(one_a, np.full((P, 64, 32), ONE_FP8, np.uint8), unit, unit)
    dC = tiles(all_a, one_b, unit, unit)
    a_row = [np.flatnonzero(dR[la * 32]) for la in range(64)]
    b_col = [np.flatnonzero(dC[lb * 32]) for lb in range(64)]
    assert all(len(x) == 16 for x in a_row + b_col), "a one-hot element must light one row/column"
    for p in range(P):      # every element of a lane lights the same row / column
        assert np.array_equal(np.flatnonzero(dR[p]), a_row[p // 32])
        assert np.array_equal(np.flatnonzero(dC[p]), b_col[p // 32])
    idx = np.arange(64)[:, None] * 32 + np.arange(32)[None, :]
    meet = np.zeros((64, 32, 16), np.int64)
    for bit in range(11):
        pat = np.where((idx >> bit) & 1, ONE_FP4, 0).astype(np.uint8)
        d = tiles(np.broadcast_to(pat, (P, 64, 32)), one_b, unit, unit)
        for p in range(P):
            meet[p // 32, p % 32] |= (d[p, b_col[p // 32]] != 0).astype(np.int64) << bit
    sa_lane = np.zeros((64, 32, 16), np.int64)
    sb_lane = np.zeros((64, 32, 16), np.int64)
    for bit in range(6):
        s = np.broadcast_to(127 + ((np.arange(64) >> bit) & 1), (P, 64)).astype(np.int32)
        da = tiles(all_a, one_b, s, unit)
        db = tiles(all_a, one_b, unit, s)
        for p in range(P):
            sa_lane[p // 32, p % 32] |= (da[p, b_col[p // 32]] == 2.0).astype(np.int64) << bit
            sb_lane[p // 32, p % 32] |= (db[p, b_col[p // 32]] == 2.0).astype(np.int64) << bit
    return dict(a_row_pos=np.array(a_row, np.int16), b_col_pos=np.array(b_col, np.int16),
                meet=meet.astype(np.int16), sa_lane=sa_lane.astype(np.int8),
                sb_lane=sb_lane.astype(np.int8))


def main():
    out = sys.argv[1] if len(sys.argv) > 1 else os.path.join(
        ROOT, "tests", "golden", "mfma_16x16x128_f4f8_layout.npz")
    import torch
    props = torch.cuda.get_device_properties(0)
    fx = measure()
    np.savez_compressed(out, device=np.array(props.gcnArchName), **fx)
    print(f"wrote {out} ({props.gcnArchName})")


if __name__ == "__main__":
    main()
