"""Size arithmetic of the largest BASELINE workload (configs[3], cfg4: 3,000,000
Gaussians at 1920x1080 with 2 % large ones), checked on the CPU before any
GPU run: K from the oracle's tile counts for the seeded scene, the bucket
bound, every workspace query the path makes, and the 32-bit index ranges the
kernels rely on.

Index types in the kernels (csrc/fgs_binning.hip, csrc/fgs_raster.hip):
* list positions, tile starts, chunk bases and point_list entries are
  uint32 and are compared against K as int64; the two-level binning casts
  list positions to int, so it runs only for K < 2^31 - 1 (use_two_level);
* level-2 chunk numbers: at most K / 512 + 257 (grid size and the cnt2 /
  base2 rows, int64 byte offsets);
* bucket_to_tile is sized by the bound B <= (K + 31 T) / 32 and indexed as
  int64 against bucket_sum; the sampled state is indexed in size_t;
* Gaussian indices are int32 (P < 2^31).
"""
import numpy as np

from fastgs_core_amd import _lib
from fastgs_core_amd import synthetic as syn

INT32_MAX = 2**31 - 1


def test_cfg4_sizes_fit_the_index_types(oracle):
    P, W, H = 3_000_000, 1920, 1080
    sc = syn.scene_config4(0, P, 3)
    cam = syn.sphere_cameras(4, 1, W, H)[0]
    inp = syn.make_inputs(sc, cam)
    pre = oracle.preprocess_fwd(inp["means3d"], inp["opacities"], inp["viewmatrix"],
                                inp["projmatrix"], inp["campos"], inp["viewspace_points"], W, H,
                                cam.tan_fovx, cam.tan_fovy, 3, dc=inp["dc"], sh=inp["sh"],
                                scales=inp["scales"], rotations=inp["rotations"])
    tiles = pre["tiles_touched"].astype(np.int64)
    K = int(tiles.sum())
    gx, gy = (W + 15) // 16, (H + 15) // 16
    T = gx * gy
    # the workload is the stress case BASELINE describes
    assert K > 30_000_000 and tiles.max() == T
    # K fits uint32 (point_offsets is a u32 scan) and the two-level bound
    assert K < INT32_MAX
    # super-tiles (8x8 tiles) of the two-level path: at most 256
    assert ((gx + 7) // 8) * ((gy + 7) // 8) <= 256
    B_bound = (K + 31 * T) // 32
    assert B_bound < INT32_MAX and B_bound * 256 < 2**63
    # level-2 chunks: grid and per-chunk tables
    max_chunks = K // 512 + 256 + 1
    assert max_chunks < 2**31 and max_chunks * 64 < 2**32

    lib = _lib.load()
    ws = int(lib.fgs_binning_workspace_bytes(P, K, T))
    dws = int(lib.fgs_depth_order_workspace_bytes(P))
    sws = int(lib.fgs_scan_workspace_bytes(P))
    # the binning workspace holds the depth order, the level-1 list and masks
    # (12 bytes per duplicate) and the level-2 chunk tables
    assert ws >= dws + 12 * K + 2 * max_chunks * 64 * 4
    assert ws < 12 * K + 4096 * P + (1 << 30), ws  # no runaway term
    assert ws % 256 == 0 and dws % 256 == 0 and sws % 256 == 0
    assert dws >= 12 * P and sws >= 8 * (P // 4096)
    # monotone in K and P
    assert int(lib.fgs_binning_workspace_bytes(P, K + 4096, T)) >= ws
    assert int(lib.fgs_binning_workspace_bytes(P + 4096, K, T)) >= ws
    # device memory of one cfg4 frame, forward and backward: outputs, binning
    # workspace and the per-Gaussian arrays; far below 288 GB of HBM
    per_gaussian = 4 * (3 + 3 + 45 + 1 + 3 + 4 + 4) * 3  # inputs, outputs, gradients
    frame = 12 * K + ws + per_gaussian * P + 4 * B_bound + 64 * W * H
    assert frame < 16 * 2**30, frame
