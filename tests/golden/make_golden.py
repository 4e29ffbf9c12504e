"""Write the golden fixtures used by the parity tests.

Run once in the build container (it reads data files under /root/reference,
which does not exist on the GPU box):

    python tests/golden/make_golden.py

Outputs, all data only:

* ``known_answers.json``: known-answer cases transcribed from the reference's
  own tests and README (each case cites its source file:line).  Expected
  values are the literals those tests assert, or hand derivations stated next
  to the case.
* ``pointnet2_parity.json``: the two three_nn/three_interpolate fixtures of
  tools/pointnet2parity.py.  Inputs are rebuilt here from the recipe at
  tools/pointnet2parity.py:125-171 (literal binary fractions and a stdlib
  ``random.Random(20261001)`` stream); expected outputs are copied from the
  reference's recorded runs docs/parity/pointnet2-mps-safe.json (Metal) and
  docs/parity/pointnet2-cuda.json (original CUDA extension).
* ``segmentation_selections.npz``: the cloud xyz of
  docs/parity/pointnet2-segmentation-synthetic-fixture.npz and the 12 index
  arrays (4 FPS, 4 ball query, 4 three_nn) that the reference recorded on
  Metal (…-mps-safe.npz) and on the original CUDA extension (…-cuda.npz).

The reference's Python code is not imported or run.
"""

from __future__ import annotations

import json
import random
import struct
from pathlib import Path

import numpy as np

REF = Path("/root/reference")
OUT = Path(__file__).resolve().parent

NAN = "nan"
INF = "inf"
NINF = "-inf"


def f32(x: float) -> float:
    return struct.unpack("<f", struct.pack("<f", x))[0]


def nextafter32(x: float, toward: float) -> float:
    return float(np.nextafter(np.float32(x), np.float32(toward)))


def known_answers() -> list[dict]:
    cases: list[dict] = []

    def add(**case):
        cases.append(case)

    # ------------------------------------------------------------------ FPS
    add(op="fps", name="readme_square", source="README.md:82-91",
        xyz=[[[0, 0, 0], [1, 0, 0], [0, 1, 0], [1, 1, 0]]], npoint=2, start_idx=0,
        skip=False, expect=[[0, 3]])
    # tests/test_fps.py:46-48 compares against the reference; the expected list
    # is derived by hand: start 0; min d2 [0,1,1,1,1,1] -> 1; after (1,0,0)
    # [0,0,0,1,1,1] -> 3; after (-1,0,0) [0,0,0,0,1,1] -> 4; after (0,1,0) all
    # zero -> first index 0, then 0 again (exhaustion repeats index 0).
    add(op="fps", name="duplicate_points_ties", source="tests/test_fps.py:45-48",
        xyz=[[[0, 0, 0], [1, 0, 0], [1, 0, 0], [-1, 0, 0], [0, 1, 0], [0, 1, 0]]],
        npoint=6, start_idx=0, skip=False, expect=[[0, 1, 3, 4, 0, 0]])
    add(op="fps", name="all_near_origin_repeats_start", source="tests/test_compat.py:114-118",
        xyz=[[[0, 0, 0]] * 50], npoint=5, start_idx=0, skip=True, expect=[[0, 0, 0, 0, 0]])
    # Hand derivation: 3 points on a line; from start 1 the farthest is 2
    # (d2 4 vs 1), then 0; exhausted -> 0.
    add(op="fps", name="start_idx_line", source="derived (reference.py:51-57)",
        xyz=[[[0, 0, 0], [1, 0, 0], [3, 0, 0]]], npoint=4, start_idx=1, skip=False,
        expect=[[1, 2, 0, 0]])
    add(op="fps_flat", name="flat_global_indices", source="tests/test_flat.py:20-23",
        x=[[0, 0, 0], [2, 0, 0], [5, 0, 0], [10, 0, 0], [12, 0, 0]],
        ptr=[0, 3, 3, 5], out_ptr=[0, 2, 2, 3], starts=[0, 0, 0], expect=[0, 2, 3])
    add(op="fps_flat", name="flat_default_ratio", source="tests/test_flat.py:27-29",
        x=[[0, 0, 0], [1, 0, 0], [4, 0, 0]], ptr=[0, 3], out_ptr=[0, 2], starts=[0],
        expect=[0, 2])

    # ------------------------------------------------------------------ kNN
    add(op="knn", name="readme_square", source="README.md:82-92",
        query=[[[0, 0, 0], [1, 1, 0]]], ref=[[[0, 0, 0], [1, 0, 0], [0, 1, 0], [1, 1, 0]]],
        k=2, expect_idx=[[[0, 1], [3, 1]]], expect_dist=[[[0.0, 1.0], [0.0, 1.0]]])
    # tests/test_knn.py:70-74: every third point is at distance sqrt(3); the
    # 150 nearest are the first 150 indices not divisible by 3, all at 0.
    ref = [[1.0, 1.0, 1.0] if j % 3 == 0 else [0.0, 0.0, 0.0] for j in range(300)]
    ties = [j for j in range(300) if j % 3][:150]
    add(op="knn", name="ties_smaller_index", source="tests/test_knn.py:70-74",
        query=[[[0, 0, 0], [0, 0, 0]]], ref=[ref], k=150,
        expect_idx=[[ties, ties]], expect_dist=[[[0.0] * 150, [0.0] * 150]])
    x = [[0.0] * 64 for _ in range(3)]
    x[0][0], x[1][0], x[2][0] = 1.0, 1e30, 2.0
    y = [[0.0] * 64 for _ in range(2)]
    y[1][0] = NAN
    add(op="knn", name="feature_nonfinite_overflow", source="tests/test_feature_knn.py:121-136",
        query=[y], ref=[x], k=3, expect_idx=[[[0, 2, -1], [-1, -1, -1]]],
        expect_dist=[[[1.0, 2.0, INF], [INF, INF, INF]]])
    add(op="knn_flat", name="feature_nonfinite_overflow_flat", source="tests/test_feature_knn.py:135",
        x=x, y=y, batch_x=None, batch_y=None, k=3, expect=[[0, 0], [0, 2]])
    xf = [[0.0] * 64 for _ in range(5)]
    for i, v in enumerate([0.0, 1.0, 4.0, 10.0, 11.0]):
        xf[i][0] = v
    yf = [list(xf[0]), list(xf[3])]
    yf = [[v + 0.1 for v in row] for row in yf]
    add(op="knn_flat", name="feature_batches", source="tests/test_feature_knn.py:139-148",
        x=xf, y=yf, batch_x=[0, 0, 0, 1, 1], batch_y=[0, 1], k=2,
        expect=[[0, 0, 1, 1], [0, 1, 3, 4]])
    bip_x = [[0, 0, 0], [2, 0, 0], [5, 0, 0], [10, 0, 0], [12, 0, 0]]
    bip_y = [[1, 0, 0], [0, 0, 0], [11, 0, 0], [15, 0, 0]]
    add(op="knn_flat", name="bipartite", source="tests/test_flat.py:10-53",
        x=bip_x, y=bip_y, batch_x=[0, 0, 0, 2, 2], batch_y=[0, 1, 2, 2], k=2,
        expect=[[0, 0, 2, 2, 3, 3], [0, 1, 3, 4, 4, 3]])
    add(op="knn_flat", name="excludes_nonfinite", source="tests/test_flat.py:57-66",
        x=[[0, 0, 0], [NAN, 0, 0], [INF, 0, 0]], y=[[0, 0, 0], [NAN, 0, 0]],
        batch_x=None, batch_y=None, k=3, expect=[[0], [0]])
    add(op="knn_flat", name="compat_positional", source="tests/test_compat.py:69-77",
        x=[[0, 0, 0], [1, 0, 0], [10, 0, 0]], y=[[0.1, 0, 0], [10.1, 0, 0]],
        batch_x=[0, 0, 1], batch_y=[0, 1], k=1, expect=[[0, 1], [0, 2]])
    refs = [[0.0, 0.0, 0.0] for _ in range(69)]
    for j in range(66):
        refs[j][0] = j + 100.0
    refs[0][0], refs[1][0] = -1.0, 1.0
    refs[66][0], refs[67][0], refs[68][0] = 7.0, 8.0, 9.0
    queries = [[0.0, 0.0, 0.0] for _ in range(10)]
    queries[-1][0] = 8.0
    # Hand derivation for the 9 queries at the origin: nearest are 0 (-1) and
    # 1 (+1) tied at d2 1 (index order), then 100 (idx 2) and 101 (idx 3);
    # the last query at 8 sees refs 66..68 at 7, 8, 9 -> 67, 66, 68.
    add(op="knn_flat", name="ragged_ties_missing", source="tests/test_flat_ragged_mps.py:52-65",
        x=refs, y=queries, batch_x=[0] * 66 + [2] * 3, batch_y=[0] * 9 + [2], k=4,
        expect=[[q for q in range(9) for _ in range(4)] + [9, 9, 9],
                [0, 1, 2, 3] * 9 + [67, 66, 68]])

    # ------------------------------------------------------------ ball query
    add(op="ball_query", name="api_padding", source="tests/test_ball_query_api.py:11-31",
        query=[[[0, 0, 0], [0, 0, 0]]], ref=[[[0.25, 0, 0], [2.0, 0, 0]]], radius=1.0, k=3,
        expect_idx=[[[0, -1, -1], [0, -1, -1]]],
        expect_dist=[[[0.0625, 0, 0], [0.0625, 0, 0]]], compat=[[[0, 0, 0], [0, 0, 0]]])
    add(op="ball_query", name="first_k_not_nearest", source="tests/test_ball_query_mps.py:83-95",
        query=[[[0, 0, 0]]], ref=[[[0.8, 0, 0], [0.1, 0, 0], [1.0, 0, 0], [0.2, 0, 0]]],
        radius=1.0, k=2, expect_idx=[[[0, 1]]],
        expect_dist=[[[f32(f32(0.8) * f32(0.8)), f32(f32(0.1) * f32(0.1))]]])
    positions = [0, 1, 31, 32, 64, 128, 224, 250, 256]
    line = [[float(j), 0.0, 0.0] for j in range(257)]
    for k in (1, 7, 31, 33, 65):
        exp_i, exp_d = [], []
        for c in positions:
            hits = [j for j in range(257) if abs(c - j) < 20.5][:k]
            exp_i.append(hits + [-1] * (k - len(hits)))
            exp_d.append([float((c - j) ** 2) for j in hits] + [0.0] * (k - len(hits)))
        add(op="ball_query", name=f"sorted_line_k{k}", source="tests/test_ball_query_mps.py:98-124",
            query=[[line[c] for c in positions]], ref=[line], radius=20.5, k=k,
            expect_idx=[exp_i], expect_dist=[exp_d])
    pts = [[2.0, 2.0, 2.0] for _ in range(97)]
    for j in (0, 31, 32, 63, 64, 95, 96):
        pts[j] = [0.0, 0.0, 0.0]
    pts[31] = [NAN, 0.0, 0.0]
    pts[64] = [INF, 0.0, 0.0]
    add(op="ball_query", name="nonfinite_blocks_partial", source="tests/test_ball_query_mps.py:216-227",
        query=[[[0, 0, 0]]], ref=[pts], radius=0.5, k=7,
        expect_idx=[[[0, 32, 63, 95, 96, -1, -1]]], expect_dist=[[[0.0] * 7]])
    one = 1.0
    add(op="ball_query", name="exact_boundary_r1", source="tests/test_ball_query_mps.py:230-245",
        query=[[[0, 0, 0]]],
        ref=[[[nextafter32(one, 0), 0, 0], [1.0, 0, 0], [nextafter32(one, 2), 0, 0]]],
        radius=1.0, k=3, expect_idx=[[[0, -1, -1]]], expect_dist=None)
    add(op="ball_query", name="radius_sq_from_f32_radius", source="tests/test_ball_query_mps.py:248-261",
        query=[[[0, 0, 0]]], ref=[[[0.09999999403953552, 3.112176273134537e-05, 0.0]]],
        radius=0.1, k=1, expect_idx=[[[0]]], expect_dist_bits=[[[0x3C23D70A]]])
    r = 2.0 ** -62
    small, large = 0.25 * r, 0.98 * r
    add(op="ball_query", name="small_normal_radius_subnormal_terms",
        source="tests/test_ball_query_mps.py:264-285",
        query=[[[0, 0, 0]]],
        ref=[[[small, large, 0], [0, small, large], [large, 0, small],
              [small, 0.8 * r, 0], [0, small, 0.8 * r], [0.8 * r, 0, small]]],
        radius=r, k=6, expect_idx=[[[3, 4, 5, -1, -1, -1]]], expect_dist=None)
    add(op="ball_query", name="nan_inf_never_match", source="tests/test_ball_query_mps.py:435-462",
        query=[[[0, 0, 0], [NAN, 0, 0], [INF, 0, 0], [NINF, 0, 0]]],
        ref=[[[NAN, 0, 0], [INF, 0, 0], [NINF, 0, 0], [0.25, 0, 0], [0.5, 0, 0]]],
        radius=1.0, k=3,
        expect_idx=[[[3, 4, -1], [-1, -1, -1], [-1, -1, -1], [-1, -1, -1]]],
        expect_dist=[[[0.0625, 0.25, 0.0], [0, 0, 0], [0, 0, 0], [0, 0, 0]]],
        grad_out=None, expect_grad_q_row0=[-1.5, 0.0, 0.0],
        expect_grad_p=[[0, 0, 0], [0, 0, 0], [0, 0, 0], [0.5, 0, 0], [1.0, 0, 0]])
    add(op="ball_query", name="distance_gradients_padding", source="tests/test_ball_query_mps.py:465-477",
        query=[[[0, 0, 0]]], ref=[[[0.2, 0, 0], [0.5, 0, 0], [4.0, 0, 0]]], radius=1.0, k=3,
        expect_idx=[[[0, 1, -1]]], expect_dist=None, grad_out=[[[2.0, 3.0, 99.0]]],
        expect_grad_q=[[[-3.8, 0, 0]]], expect_grad_p=[[[0.8, 0, 0], [3.0, 0, 0], [0, 0, 0]]])
    add(op="ball_query", name="repeated_point_accumulates", source="tests/test_ball_query_mps.py:513-525",
        query=[[[0, 0, 0], [1.0, 0, 0]]], ref=[[[0.25, 0, 0]]], radius=2.0, k=1,
        expect_idx=[[[0], [0]]], expect_dist=None, grad_out=[[[2.0], [3.0]]],
        expect_grad_q=[[[-1.0, 0, 0], [4.5, 0, 0]]], expect_grad_p=[[[-3.5, 0, 0]]])
    add(op="ball_query", name="invalid_slots_do_not_poison", source="tests/test_ball_query_mps.py:498-510",
        query=[[[0, 0, 0]]], ref=[[[NAN, 0, 0], [0.25, 0, 0]]], radius=1.0, k=3,
        expect_idx=[[[1, -1, -1]]], expect_dist=None, grad_out=[[[1.0, 99.0, NAN]]],
        expect_grad_q=[[[-0.5, 0, 0]]], expect_grad_p=[[[0, 0, 0], [0.5, 0, 0]]])
    add(op="ball_query", name="empty_missing_nonfinite", source="tests/test_ball_query_mps.py:566-571",
        query=[[[0, 0, 0], [2.0, 0, 0]]], ref=[[[NAN, 0, 0], [0.1, 0, 0]]], radius=0.5, k=3,
        expect_idx=[[[1, -1, -1], [-1, -1, -1]]], expect_dist=None)
    add(op="ball_query", name="readme_square", source="README.md:82-93",
        query=[[[0, 0, 0], [1, 1, 0]]], ref=[[[0, 0, 0], [1, 0, 0], [0, 1, 0], [1, 1, 0]]],
        radius=1.1, k=2, expect_idx=[[[0, 1], [1, 2]]], expect_dist=[[[0, 1], [1, 1]]])
    add(op="ball_query", name="compat_first_hit_padding", source="tests/test_compat.py:140-145",
        query=[[[0, 0, 0], [50, 50, 50]]], ref=[[[5.0, 0, 0], [0.1, 0, 0], [9, 9, 9], [0.2, 0, 0]]],
        radius=0.5, k=4, expect_idx=[[[1, 3, -1, -1], [-1, -1, -1, -1]]], expect_dist=None,
        compat=[[[1, 3, 1, 1], [0, 0, 0, 0]]])
    # reference.py:102-121 with r = 1e20: r2 = fl32(1e40) = inf, so every
    # finite d2 is a hit and an overflowed d2 (5e19^2) is not: [[0, -1, -1]].
    # (The reference's Metal kernel takes a normalised path here and also
    # accepts index 1; this build follows reference.py.)
    add(op="ball_query", name="huge_radius_overflow", source="reference.py:83-121 (r2 = inf)",
        query=[[[0, 0, 0]]], ref=[[[1e19, 0, 0], [5e19, 0, 0], [2e20, 0, 0]]], radius=1e20, k=3,
        expect_idx=[[[0, -1, -1]]], expect_dist=None)
    add(op="ball_query", name="zero_radius", source="tests/test_ball_query_api.py:53-57",
        query=[[[0, 0, 0], [0.5, 0.5, 0.5]]], ref=[[[0, 0, 0], [0.5, 0.5, 0.5], [1, 1, 1]]],
        radius=0.0, k=3, expect_idx=[[[-1, -1, -1], [-1, -1, -1]]],
        expect_dist=[[[0, 0, 0], [0, 0, 0]]])
    add(op="radius_flat", name="bipartite_strict", source="tests/test_flat.py:69-73",
        x=bip_x, y=bip_y, batch_x=[0, 0, 0, 2, 2], batch_y=[0, 1, 2, 2], r=1.1, k=2,
        expect=[[0, 0, 2, 2], [0, 1, 3, 4]])
    add(op="radius_flat", name="boundary_strict", source="tests/test_flat.py:74",
        x=bip_x[:2], y=bip_x[:1], batch_x=None, batch_y=None, r=1.0, k=32,
        expect=[[0], [0]])
    add(op="radius_flat", name="cap_one", source="tests/test_flat.py:75-77",
        x=bip_x, y=bip_y, batch_x=[0, 0, 0, 2, 2], batch_y=[0, 1, 2, 2], r=100.0, k=1,
        expect=[[0, 2, 3], [0, 3, 3]])
    add(op="radius_flat", name="torch_cluster_threshold_r021", source="tests/test_flat.py:207-217",
        x=[[f32(0.21), 0, 0]], y=[[0, 0, 0]], batch_x=None, batch_y=None, r=0.21, k=32,
        expect=[[0], [0]])
    add(op="radius_flat", name="torch_cluster_threshold_r01", source="tests/test_flat.py:219-224",
        x=[[f32(0.1), 0, 0]], y=[[0, 0, 0]], batch_x=None, batch_y=None, r=0.1, k=32,
        expect=[[], []])
    add(op="radius_flat", name="discards_nonfinite", source="tests/test_flat_ragged_mps.py:38-49",
        x=[[0, 0, 0], [NAN, 0, 0], [0.25, 0, 0], [INF, 0, 0]],
        y=[[0, 0, 0], [NAN, 0, 0], [INF, 0, 0]], batch_x=None, batch_y=None, r=1.0, k=4,
        expect=[[0, 0], [0, 2]])
    rr = [[20.0, 20.0, 20.0] for _ in range(75)]
    for j in (3, 31, 32, 33, 63, 64, 69):
        rr[j] = [0.25, 0.0, 0.0]
    for j in range(70, 75):
        rr[j] = [10.0, 0.0, 0.0]
    qq = [[0.0, 0.0, 0.0] for _ in range(9)] + [[10.0, 0.0, 0.0]]
    add(op="radius_flat", name="first_k_across_blocks", source="tests/test_flat_ragged_mps.py:21-35",
        x=rr, y=qq, batch_x=[0] * 70 + [2] * 5, batch_y=[0] * 9 + [2], r=1.0, k=4,
        expect=[[q for q in range(9) for _ in range(4)] + [9] * 4,
                [3, 31, 32, 33] * 9 + [70, 71, 72, 73]])
    line3 = [[0.0, 0.0, 0.0], [1.0, 0.0, 0.0], [2.0, 0.0, 0.0]]
    add(op="radius_flat", name="graph_loop_self", source="tests/test_flat_graph.py:8-22",
        x=line3, y=line3, batch_x=None, batch_y=None, r=1.1, k=2,
        expect=[[0, 0, 1, 1, 2, 2], [0, 1, 0, 1, 1, 2]])

    # ------------------------------------------------------------ three_nn
    add(op="three_nn", name="order_ties", source="tests/test_pointnet2.py:24-39",
        unknown=[[[0, 0, 0], [2, 0, 0]]], known=[[[1, 0, 0], [-1, 0, 0], [0, 2, 0], [1, 0, 0]]],
        expect_idx=[[[0, 1, 3], [0, 3, 2]]],
        expect_dist=[[[1, 1, 1], [1, 1, 2.8284271247461903]]])
    add(op="three_interpolate", name="repeated_indices", source="tests/test_pointnet2.py:72-90",
        features=[[[2, 3, 5, 7], [11, 13, 17, 19]]], indices=[[[0, 1, 1], [3, 1, 0]]],
        weights=[[[0.5, 0.25, 0.25], [1, 0.5, -0.5]]], expect=[[[2.5, 7.5], [12, 20]]],
        grad_out=[[[1, 1], [1, 1]]], expect_grad=[[[0, 1, 0, 1], [0, 1, 0, 1]]])

    # -------------------------------------------------------------- Chamfer
    add(op="chamfer_nearest", name="tie_first_index", source="tests/test_chamfer.py:8-20",
        query=[[[1, 0, 0]]], ref=[[[0, 0, 0], [2, 0, 0]]], norm=2, expect_idx=[[0]],
        expect_dist=[[1.0]])
    add(op="chamfer_nearest", name="overflow_keeps_first", source="tests/test_chamfer.py:178-192",
        query=[[[1e20, 0, 0]]], ref=[[[0, 0, 0], [1, 0, 0]]], norm=2, expect_idx=[[0]],
        expect_dist=[[INF]])
    add(op="chamfer_nearest", name="l1_tie_padding", source="tests/test_chamfer.py:229-241",
        query=[[[0, 0, 0], [NAN, 0, 0]]], ref=[[[1, 0, 0], [-1, 0, 0]]], norm=1,
        query_lengths=[1], ref_lengths=[2], expect_idx=[[0, -1]], expect_dist=[[1.0, 0.0]])
    qz = [[0.0, 0.0, 0.0] for _ in range(17)]
    rf = [[100.0, 100.0, 100.0] for _ in range(65)]
    rf[0], rf[31], rf[32], rf[64] = [1.0, 0, 0], [-1.0, 0, 0], [0, 1.0, 0], [0, -1.0, 0]
    add(op="chamfer_nearest", name="l1_tie_across_lanes", source="tests/test_chamfer.py:267-282",
        query=[qz, qz], ref=[rf, rf], norm=1, expect_idx=[[0] * 17, [0] * 17],
        expect_dist=[[1.0] * 17, [1.0] * 17])
    qn = [[[0.0, 0.0, 0.0] for _ in range(9)] for _ in range(2)]
    qn[0][8] = [NAN, 0, 0]
    qn[1][7] = [NAN, 0, 0]
    qn[1][8] = [NAN, 0, 0]
    rn = [[[9.0, 9.0, 9.0] for _ in range(37)] for _ in range(2)]
    for b in range(2):
        rn[b][0], rn[b][31], rn[b][36] = [1.0, 0, 0], [-1.0, 0, 0], [0, 1.0, 0]
    add(op="chamfer_nearest", name="writes_every_row_first_tie", source="tests/test_chamfer.py:452-477",
        query=qn, ref=rn, norm=2, query_lengths=[8, 7], ref_lengths=[37, 32],
        expect_idx=[[0] * 8 + [-1], [0] * 7 + [-1, -1]],
        expect_dist=[[1.0] * 8 + [0.0], [1.0] * 7 + [0.0, 0.0]])
    for dim in (1, 2, 4, 64, 128):
        for norm in (1, 2):
            y2 = [[0.0] * dim, [0.0] * dim]
            y2[0][0], y2[1][0] = 1.0, -1.0
            add(op="chamfer_nearest", name=f"nd_first_tie_d{dim}_n{norm}",
                source="tests/test_chamfer_nd.py:50-73",
                query=[[[0.0] * dim]], ref=[y2], norm=norm, expect_idx=[[0]], expect_dist=[[1.0]])
            y3 = [[0.0] * dim, [0.0] * dim]
            y3[0][0], y3[1][0] = 1e30, -1e30
            add(op="chamfer_nearest", name=f"nd_overflow_first_d{dim}_n{norm}",
                source="tests/test_chamfer_nd.py:76-95",
                query=[[[0.0] * dim, [0.0] * dim]], ref=[y3], norm=norm,
                query_lengths=[1], ref_lengths=[2], expect_idx=[[0, -1]],
                expect_dist=[[f32(1e30) if norm == 1 else INF, 0.0]])
    return cases


def pointnet2_parity() -> dict:
    """Inputs per tools/pointnet2parity.py:125-171; outputs from docs/parity."""
    small = {
        "known": [
            [[-1, 0, 0], [1, 0, 0], [0, -1, 0], [0, 1, 0], [0, 0, 1], [0, 0, -1]],
            [[2, 0, 0], [2, 1, 0], [2, -1, 0], [3, 0, 0], [1, 0, 0], [2, 0, 1]],
        ],
        "unknown": [
            [[0, 0, 0], [0.25, 0.125, 0], [-0.5, 0.25, 0.125], [0, 0, 0.75]],
            [[2, 0, 0], [2.25, 0.125, 0], [1.5, -0.25, 0.125], [2, 0, 0.75]],
        ],
        "features": [
            [[1, 2, 3, 4, 5, 6], [-0.5, 0.25, 1.5, -2, 2.5, 3.25]],
            [[3, 1, -1, 2, 4, -2], [0.125, -0.25, 0.5, 1, -1.5, 2]],
        ],
        "weights": [
            [[0.5, 0.25, 0.25], [0.125, 0.375, 0.5], [0.25, 0.5, 0.25], [0.75, 0.125, 0.125]],
            [[0.25, 0.5, 0.25], [0.5, 0.25, 0.25], [0.375, 0.125, 0.5], [0.125, 0.75, 0.125]],
        ],
        "gradient": [
            [[1, 0.25, -0.5, 0.125], [0.5, -1, 0.25, 0.75]],
            [[-0.25, 1.5, 0.5, -1], [1, 0.125, -0.75, 0.25]],
        ],
        # tools/pointnet2parity.py:187-189 overrides the interpolation indices
        # of query 0 in each batch after three_nn.
        "override": {"0": [1, 1, 2], "1": [3, 3, 3]},
    }
    rng = random.Random(20261001)

    def point():
        return [rng.randint(-10000, 10000) / 1024 for _ in range(3)]

    known = [[point() for _ in range(257)]]
    unknown = [[point() for _ in range(73)]]
    features = [[[rng.randint(-2048, 2048) / 1024 for _ in range(257)] for _ in range(5)]]
    weights = [[[rng.randint(0, 1024) / 1024 for _ in range(3)] for _ in range(73)]]
    gradient = [[[rng.randint(-1024, 1024) / 1024 for _ in range(73)] for _ in range(5)]]
    large = {"known": known, "unknown": unknown, "features": features, "weights": weights,
             "gradient": gradient, "override": {}}
    out = {"source": "tools/pointnet2parity.py:125-171; docs/parity/pointnet2-{mps-safe,cuda}.json",
           "cases": {"ties-and-duplicates": {"inputs": small}, "seeded-stride": {"inputs": large}}}
    for backend, fname in (("mps_safe", "pointnet2-mps-safe.json"), ("cuda", "pointnet2-cuda.json")):
        rec = json.loads((REF / "docs" / "parity" / fname).read_text())
        for case, data in rec["cases"].items():
            out["cases"][case][backend] = {
                key: data[key] for key in ("nearest_indices", "distances", "interpolate_indices",
                                           "interpolated", "feature_gradient", "weight_gradient")
            }
    return out


def segmentation() -> dict[str, np.ndarray]:
    parity = REF / "docs" / "parity"
    fixture = np.load(parity / "pointnet2-segmentation-synthetic-fixture.npz", allow_pickle=False)
    arrays = {"xyz": np.ascontiguousarray(fixture["points"][..., :3]).astype(np.float32)}
    for tag, fname in (("mps", "pointnet2-segmentation-mps-safe.npz"),
                       ("cuda", "pointnet2-segmentation-cuda.npz")):
        data = np.load(parity / fname, allow_pickle=False)
        for key in data.files:
            if key.startswith("selection::"):
                arrays[f"{tag}::{key[len('selection::'):]}"] = data[key].astype(np.int32)
    return arrays


def main() -> None:
    cases = known_answers()
    (OUT / "known_answers.json").write_text(json.dumps({"cases": cases}, indent=None) + "\n")
    (OUT / "pointnet2_parity.json").write_text(json.dumps(pointnet2_parity()) + "\n")
    np.savez_compressed(OUT / "segmentation_selections.npz", **segmentation())
    print(f"wrote {len(cases)} known-answer cases")


if __name__ == "__main__":
    main()
