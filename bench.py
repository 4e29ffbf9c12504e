"""Benchmark of the neighbourhood-search hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

North-star workload ("PointNet++ MSG layer"): B=32
clouds of N=4096 points on 1-4 noisy spheres; one step is

    FPS npoint=1024 -> ball_query(r, K) for (0.1,16), (0.2,32), (0.4,128)
    -> knn(centres, cloud, 16)

and the metric is points/s = B*N / (t_FPS + sum t_ball + t_kNN), inputs
resident in HBM.  Prints one JSON line with the roofline of the dominant kernel
(timed with HIP events on the launch stream) and the CPU baseline (this
build's PyTorch-CPU port of the reference's algorithms, oracle/torch_port.py,
on a bounded sample of the same workload).

The input generators for all five BASELINE.json configs live here so the
tests build exactly the benchmarked data.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import subprocess
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "mps-pointops_amd"))

# ------------------------------------------------------------- workloads


def make_c1(seed: int = 1) -> torch.Tensor:
    """Config 1: B=16, N=1024 uniform in [-1,1]^3."""
    g = torch.Generator().manual_seed(seed)
    return 2 * torch.rand(16, 1024, 3, generator=g) - 1


def make_c2(seed: int = 2, B: int = 32, N: int = 4096) -> torch.Tensor:
    """Config 2: per cloud 1-4 spheres (radius U[0.2,0.8], centre U[-0.5,0.5]^3),
    points split evenly over the spheres, on-sphere by normalised randn, plus
    N(0, 0.01) noise."""
    g = torch.Generator().manual_seed(seed)
    clouds = []
    for _ in range(B):
        ns = int(torch.randint(1, 5, (1,), generator=g))
        radii = 0.2 + 0.6 * torch.rand(ns, generator=g)
        centres = torch.rand(ns, 3, generator=g) - 0.5
        counts = [N // ns + (1 if i < N % ns else 0) for i in range(ns)]
        parts = []
        for s in range(ns):
            d = torch.randn(counts[s], 3, generator=g)
            d = d / d.norm(dim=1, keepdim=True).clamp_min(1e-12)
            parts.append(centres[s] + radii[s] * d)
        cloud = torch.cat(parts) + 0.01 * torch.randn(N, 3, generator=g)
        clouds.append(cloud)
    return torch.stack(clouds).float().contiguous()


def make_c3(seed: int = 3, N: int = 1 << 20) -> torch.Tensor:
    """Config 3: one LiDAR-like slab, x,y in [-50,50]^2 accepted with
    probability 1/(1+r^2), z U[0,4]."""
    g = torch.Generator().manual_seed(seed)
    out = []
    have = 0
    while have < N:
        xy = torch.rand(1 << 22, 2, generator=g, dtype=torch.float64) * 100 - 50
        r2 = (xy * xy).sum(1)
        keep = torch.rand(1 << 22, generator=g, dtype=torch.float64) < 1.0 / (1.0 + r2)
        xy = xy[keep]
        out.append(xy)
        have += len(xy)
    xy = torch.cat(out)[:N]
    z = torch.rand(N, 1, generator=g, dtype=torch.float64) * 4
    return torch.cat([xy, z], 1).float().unsqueeze(0).contiguous()


def make_c4_clustered(seed: int = 41) -> tuple[torch.Tensor, torch.Tensor]:
    """Config 4's sizes on clustered data: 1,048,576 references in 40 tight
    Gaussian clusters (sigma 0.1) at uniform centres in [0,100]^3, and 131072
    queries uniform over the same box, so most queries lie far from every
    reference (the grid search's worst case)."""
    g = torch.Generator().manual_seed(seed)
    n = 1 << 20
    centres = torch.rand(40, 3, generator=g) * 100
    ref = centres.repeat_interleave(n // 40 + 1, 0)[:n] + torch.randn(n, 3, generator=g) * 0.1
    query = torch.rand(131072, 3, generator=g) * 100
    return ref[None].contiguous(), query[None].contiguous()


def make_c4(seed: int = 4) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Config 4: ref 1,048,576 and 131,072 queries uniform in [0,10]^3, plus
    DGCNN features randn(8, 2048, 64)."""
    g = torch.Generator().manual_seed(seed)
    ref = torch.rand(1, 1 << 20, 3, generator=g) * 10
    query = torch.rand(1, 131072, 3, generator=g) * 10
    feat = torch.randn(8, 2048, 64, generator=g)
    return ref, query, feat


def make_c5(seed: int = 5, B: int = 32, P: int = 8192) -> tuple[torch.Tensor, torch.Tensor]:
    """Config 5: y1 on the unit sphere, y2 = y1 + N(0,0.02) with 10% of points
    (first floor(0.1P) of a seeded permutation) replaced by U[-1,1]^3."""
    g = torch.Generator().manual_seed(seed)
    y1 = torch.randn(B, P, 3, generator=g)
    y1 = y1 / y1.norm(dim=-1, keepdim=True).clamp_min(1e-12)
    y2 = y1 + 0.02 * torch.randn(B, P, 3, generator=g)
    m = P // 10
    for b in range(B):
        sel = torch.randperm(P, generator=g)[:m]
        y2[b, sel] = torch.rand(m, 3, generator=g) * 2 - 1
    return y1.contiguous(), y2.contiguous()


C2_RADII = ((0.1, 16), (0.2, 32), (0.4, 128))
C2_NPOINT = 1024
C2_KNN_K = 16
C2_CHUNK = 128  # centres per chunk of the overlapped step (mps_pointops.fps_ball_knn)

# ---------------------------------------------------------------- timing

MI355X_HBM_BYTES_PER_S = 8.0e12
# Published MI355X vector/matrix FP32 peak.  This path runs on the FP32 VALU
# without FMA (the reference's rounding) and without packed FP32, so its own
# issue ceiling is 256 CUs x 64 lanes x 2.4 GHz = 39.3 T op/s; the JSON line
# reports against the published figure.
MI355X_FP32_PEAK = 157.3e12
# Issue ceiling of unfused, unpacked FP32 VALU code: one op per lane per clock,
# 64 lanes per CU (4 SIMDs x 16), 256 CUs at 2.4 GHz.
MI355X_CUS = 256
MI355X_VALU_ISSUE_PER_CU = 64 * 2.4e9
MI355X_VALU_ISSUE = MI355X_CUS * MI355X_VALU_ISSUE_PER_CU
FPS_OPS_PER_POINT_STEP = 9  # 3 sub, 3 mul, 2 add (unfused), 1 min
PAIR_OPS = 8                # 3-D squared distance: 3 sub, 3 mul, 2 add


class KernelTimer:
    """HIP-event timing on the stream the kernels are launched on."""

    def __init__(self, stream):
        self.stream = stream

    def time(self, fn, reps: int) -> float:
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(self.stream)
        for _ in range(reps):
            fn()
        end.record(self.stream)
        end.synchronize()
        return start.elapsed_time(end) / 1e3 / reps


def fps_kernel_name(n: int) -> str:
    """Template instance of the dense FPS kernel that a cloud of n points
    uses: fps_lead_kernel<P> up to 4096 points (P points per follower lane),
    fps_tiled_kernel<16,512,16> up to 8192."""
    p = 1
    while p * 512 < n:
        p *= 2
    return f"fps_lead_kernel<{p}>" if p <= 8 else f"fps_tiled_kernel<{p},512,{p}>"


def profiled_traffic(kernel: str, workload: str):
    """HBM bytes per launch of `kernel` on `workload`, as recorded from the
    FETCH_SIZE/WRITE_SIZE counter runs in profiles/*.md (a line
    `traffic_bytes_per_launch[<kernel>@<workload>]: <bytes>`), else None."""
    key = f"traffic_bytes_per_launch[{kernel}@{workload}]:"
    for path in sorted((ROOT / "profiles").glob("*.md")):
        for line in path.read_text().splitlines():
            if line.strip().startswith(key):
                return float(line.split(":", 1)[1].strip())
    return None


def ball_scanned_pairs(idx: torch.Tensor, n: int) -> int:
    """Pairs a first-K ball query must test: up to the K-th hit, else all n."""
    last = idx[..., -1]
    return int(torch.where(last >= 0, last + 1, torch.full_like(last, n)).sum())


def cpu_info() -> dict:
    model = platform.processor() or ""
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return {"model": model, "os_cpu_count": os.cpu_count()}


def cpu_baseline(xyz_cpu: torch.Tensor, clouds: int, warmup: int = 3, repeats: int = 20) -> dict:
    """The reference's CPU algorithms (PyTorch-CPU port) on the first
    `clouds` clouds of the config-2 input, scaled to points/s: `warmup`
    untimed passes, then the median of `repeats` timed passes (each op's
    median reported beside the total)."""
    import statistics

    sys.path.insert(0, str(ROOT))
    from oracle import torch_port

    torch.set_num_threads(os.cpu_count() or 1)
    x = xyz_cpu[:clouds].contiguous()

    def one_pass() -> tuple[float, float, float]:
        t0 = time.perf_counter()
        idx = torch_port.furthest_point_sample(x, C2_NPOINT)
        t_fps = time.perf_counter() - t0
        centres = x.gather(1, idx[..., None].expand(-1, -1, 3))
        s = time.perf_counter()
        for radius, k in C2_RADII:
            torch_port.ball_query(centres, x, radius, k)
        t_ball = time.perf_counter() - s
        s = time.perf_counter()
        torch_port.knn(centres, x, C2_KNN_K)
        return t_fps, t_ball, time.perf_counter() - s

    for _ in range(warmup):
        one_pass()
    passes = [one_pass() for _ in range(max(1, repeats))]
    total = statistics.median(sum(p) for p in passes)
    t_fps, t_ball, t_knn = (statistics.median(p[i] for p in passes) for i in range(3))
    return {
        "value": clouds * x.shape[1] / total,
        "unit": "points/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{clouds} of 32 clouds of config 2 (N=4096): FPS 1024 + 3 ball queries + kNN16, "
                  f"PyTorch-CPU port of reference.py, median of {len(passes)} passes after "
                  f"{warmup} warmups; medians fps {t_fps:.3f}s ball {t_ball:.3f}s "
                  f"knn {t_knn:.3f}s",
        "cpu": cpu_info(),
    }


def cpu_baseline_other(config: str) -> dict:
    """The reference's CPU algorithms (PyTorch-CPU port) on a bounded sample
    of configs 1, 3, 4 and 5, scaled to the config's metric: one untimed
    pass, then the median of 3 timed passes."""
    import statistics

    sys.path.insert(0, str(ROOT))
    from oracle import torch_port

    torch.set_num_threads(os.cpu_count() or 1)

    def median_time(fn) -> float:
        fn()
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        return statistics.median(times)

    if config == "c1":
        x = make_c1()
        B, N, _ = x.shape
        c = x.gather(1, torch_port.furthest_point_sample(x, 512)[..., None].expand(-1, -1, 3))
        t_fps = median_time(lambda: torch_port.furthest_point_sample(x, 512))
        t_ball = median_time(lambda: torch_port.ball_query(c, x, 0.2, 32))
        t_knn = median_time(lambda: torch_port.knn(c, x, 16))
        value, unit = B * N / (t_fps + t_ball + t_knn), "points/s"
        sample = (f"the whole workload; medians fps {t_fps:.3f}s ball {t_ball:.3f}s "
                  f"knn {t_knn:.3f}s")
    elif config == "c3":
        x = make_c3()
        N = x.shape[1]
        steps, queries = 256, 64
        c = x[:, torch.randperm(N, generator=torch.Generator().manual_seed(3))[:queries]]
        t_fps = median_time(lambda: torch_port.furthest_point_sample(x, steps)) * 16384 / steps
        t_ball = median_time(lambda: torch_port.ball_query(c, x, 0.5, 32)) * 16384 / queries
        value, unit = N / (t_fps + t_ball), "points/s"
        sample = (f"FPS: the first {steps} of 16384 steps (x {16384 // steps}); ball query: "
                  f"{queries} of the 16384 queries over all 2^20 points (x {16384 // queries}); "
                  f"scaled fps {t_fps:.1f}s ball {t_ball:.1f}s")
    elif config == "c4":
        ref, query, _ = make_c4()
        M = query.shape[1]
        sub = 256
        t_knn = median_time(lambda: torch_port.knn(query[:, :sub], ref, 16)) * M / sub
        value, unit = M / t_knn, "queries/s"
        sample = f"{sub} of the {M} queries against all 2^20 references (x {M // sub}): {t_knn:.1f}s"
    else:
        y1, y2 = make_c5()
        B, P, _ = y1.shape
        clouds = 2

        def fwd_bwd():
            a = y1[:clouds].clone().requires_grad_()
            b = y2[:clouds].clone().requires_grad_()
            torch_port.chamfer_l2(a, b).backward()

        t = median_time(fwd_bwd) * B / clouds
        value, unit = 2 * B * P / t, "points/s"
        sample = f"{clouds} of the {B} clouds, forward + backward (x {B // clouds}): {t:.1f}s"
    return {"value": value, "unit": unit, "cores": torch.get_num_threads(), "kind": "port",
            "sample": "PyTorch-CPU port of the reference's CPU path, " + sample,
            "cpu": cpu_info()}


def timed_steps(step, steps: int, warmup: int) -> float:
    """Seconds per step over exactly `steps` steps after `warmup` untimed ones,
    synchronised on both sides."""
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def pipelined_steps(mp, xyz: torch.Tensor, steps: int, warmup: int) -> float:
    """Seconds per step of the config-2 step software-pipelined over two
    streams: step i samples batch i on one stream while the other runs the
    three ball queries and kNN on the centres of batch i-1 (waiting for
    that FPS's event).  Every step does the whole work of one batch; the
    input is the same resident cloud each time."""
    B = xyz.shape[0]
    s_fps, s_q = torch.cuda.Stream(), torch.cuda.Stream()
    done_fps = [torch.cuda.Event(), torch.cuda.Event()]
    done_q = [torch.cuda.Event(), torch.cuda.Event()]
    idx = [None, None]

    def sample(i):
        with torch.cuda.stream(s_fps):
            s_fps.wait_event(done_q[i % 2])  # batch i-2's queries are done with idx[i % 2]
            idx[i % 2] = mp.furthest_point_sample(xyz, C2_NPOINT)
            idx[i % 2].record_stream(s_q)
            done_fps[i % 2].record(s_fps)

    def query(i):
        with torch.cuda.stream(s_q):
            s_q.wait_event(done_fps[i % 2])
            centres = xyz.gather(1, idx[i % 2][..., None].expand(-1, -1, 3)).contiguous()
            for radius, k in C2_RADII:
                mp.ball_query(centres, xyz, radius, k)
            mp.knn(centres, xyz, C2_KNN_K)
            done_q[i % 2].record(s_q)

    for e in done_q:
        e.record(torch.cuda.current_stream())
    sample(0)
    for i in range(1, warmup + 1):
        sample(i)
        query(i - 1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(warmup + 1, warmup + 1 + steps):
        sample(i)
        query(i - 1)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def run(args) -> dict:
    import mps_pointops as mp

    device = torch.device("cuda", 0)
    xyz_cpu = make_c2()
    xyz = xyz_cpu.to(device)
    B, N, _ = xyz.shape
    timer = KernelTimer(torch.cuda.current_stream(device))
    state = {}

    def fps():
        state["idx"] = mp.furthest_point_sample(xyz, C2_NPOINT)

    fps()
    torch.cuda.synchronize()
    centres = xyz.gather(1, state["idx"][..., None].expand(-1, -1, 3)).contiguous()

    def balls():
        for radius, k in C2_RADII:
            mp.ball_query(centres, xyz, radius, k)

    def knn():
        mp.knn(centres, xyz, C2_KNN_K)

    def step():
        fps()
        balls()
        knn()

    wall_sequential = timed_steps(step, args.steps, args.warmup)

    # The same batch's FPS, centre gather, ball queries and kNN in one call
    # (mps_pointops.fps_ball_knn): the ball queries of each C2_CHUNK-centre chunk
    # run as soon as FPS has sampled it, on the CUs FPS leaves free, and kNN
    # once after the last chunk.  Same outputs,
    # bit for bit (tests/test_gpu_pipeline.py); this is the timed step.
    radii = [r for r, _ in C2_RADII]
    ks = [k for _, k in C2_RADII]

    def fused_step():
        state["fused"] = mp.fps_ball_knn(xyz, C2_NPOINT, radii, ks, C2_KNN_K, chunk=C2_CHUNK)

    wall = timed_steps(fused_step, args.steps, args.warmup)
    # The last timed call's outputs against the separate calls, bit for bit
    # (outside the timed region): a chunk whose wait gave up would show here.
    samples, fused_centres, fused_balls, fused_knn = state["fused"]
    same = torch.equal(samples, state["idx"]) and torch.equal(fused_centres, centres)
    for (radius, k), (d, i) in zip(C2_RADII, fused_balls):
        rd, ri = mp.ball_query(centres, xyz, radius, k)
        same = same and torch.equal(i, ri) and torch.equal(d, rd)
    kd, ki = mp.knn(centres, xyz, C2_KNN_K)
    same = same and torch.equal(fused_knn[1], ki) and torch.equal(fused_knn[0], kd)
    if not same:
        raise SystemExit("bench: fps_ball_knn's last timed call differs from the separate calls")

    # Per-op kernel time on the launch stream (HIP events).
    reps = max(5, args.steps)
    t_fps = timer.time(fps, reps)
    t_ball = timer.time(balls, reps)
    t_knn = timer.time(knn, reps)
    # The same three ball queries as one multi-radius scan (not in value).
    multi = mp.ball_query_multi(centres, xyz, radii, ks)
    for (radius, k), (d, i) in zip(C2_RADII, multi):
        rd, ri = mp.ball_query(centres, xyz, radius, k)
        if not (torch.equal(i, ri) and torch.equal(d, rd)):
            raise SystemExit("bench: ball_query_multi differs from the separate ball queries")
    t_ball_multi = timer.time(lambda: mp.ball_query_multi(centres, xyz, radii, ks), reps)

    # Algorithmic work (FP32 ops): FPS 9 per point-step; ball query 8 per
    # scanned pair (up to the K-th hit); kNN 8 per pair (all pairs).
    fps_ops = FPS_OPS_PER_POINT_STEP * B * C2_NPOINT * N
    ball_ops = sum(PAIR_OPS * ball_scanned_pairs(mp.ball_query(centres, xyz, r, k)[1], N)
                   for r, k in C2_RADII)
    knn_ops = PAIR_OPS * B * C2_NPOINT * N

    def op(t, ops):
        return {"ms": t * 1e3, "points_per_s": B * N / t, "tops": ops / t / 1e12,
                "frac_fp32_peak": ops / t / MI355X_FP32_PEAK}

    # Config 2's feature propagation (not part of the metric): three_nn from
    # the 1024 centres to the 4096 points, three_interpolate of C=128 features
    # (forward and backward), HBM bytes = inputs read once + outputs written.
    from mps_pointops import three_interpolate, three_nn

    g = torch.Generator().manual_seed(9)
    feats = torch.randn(B, 128, C2_NPOINT, generator=g).to(device)
    tn_d, tn_i = three_nn(xyz, centres)
    inv = 1.0 / (tn_d + 1e-8)
    w = (inv / inv.sum(-1, keepdim=True)).contiguous()
    upstream = torch.randn(B, 128, N, generator=g).to(device)
    fleaf = feats.clone().requires_grad_()

    def interp_fwd_bwd():
        fleaf.grad = None
        three_interpolate(fleaf, tn_i, w).backward(upstream)

    for _ in range(max(1, args.warmup)):  # first-use library loading
        three_nn(xyz, centres)
        three_interpolate(feats, tn_i, w)
        interp_fwd_bwd()
    torch.cuda.synchronize()
    t_tn = timer.time(lambda: three_nn(xyz, centres), reps)
    t_ti = timer.time(lambda: three_interpolate(feats, tn_i, w), reps)
    t_tib = timer.time(interp_fwd_bwd, reps)
    interp_bytes = 4 * (B * 128 * C2_NPOINT + 2 * B * N * 3 + B * 128 * N)
    # Set-abstraction grouping after the r=0.2 ball query (not part of the
    # metric): grouped xyz - centre and C=64 grouped features in one fused
    # kernel, forward and forward+backward (bytes = output written + index,
    # features and xyz read once).
    from mps_pointops import group as grouping
    from mps_pointops import compat

    sa_feats = torch.randn(B, 64, N, generator=g).to(device)
    sa_idx = compat.ball_query(0.2, 32, xyz, centres)
    sa_leaf = sa_feats.clone().requires_grad_()
    sa_up = torch.randn(B, 67, C2_NPOINT, 32, generator=g).to(device)

    def group_fwd():
        return grouping.query_and_group(xyz, centres, sa_feats, sa_idx, check=False)

    def group_fwd_bwd():
        sa_leaf.grad = None
        grouping.query_and_group(xyz, centres, sa_leaf, sa_idx, check=False).backward(sa_up)

    sa_layer = grouping.QueryAndGroup(0.2, 32)

    def group_layer():  # the whole layer step: ball query (pointnet2 form) + grouping
        return sa_layer(xyz, centres, sa_feats)

    group_fwd()
    group_fwd_bwd()
    group_layer()
    torch.cuda.synchronize()
    t_gf = timer.time(group_fwd, reps)
    t_gfb = timer.time(group_fwd_bwd, reps)
    t_gl = timer.time(group_layer, reps)
    group_bytes = 4 * (B * 67 * C2_NPOINT * 32 + B * C2_NPOINT * 32 + B * 64 * N + B * N * 3)
    # Ball query with gradients (r=0.4, K=128, the largest of the three): the
    # forward alone and forward + backward (both coordinate gradients).
    bq_q = centres.clone().requires_grad_()
    bq_p = xyz.clone().requires_grad_()
    bq_g = torch.randn(B, C2_NPOINT, 128, generator=g).to(device)

    def ball_fwd():
        return mp.ball_query(bq_q, bq_p, 0.4, 128)

    def ball_fwd_bwd():
        bq_q.grad = None
        bq_p.grad = None
        mp.ball_query(bq_q, bq_p, 0.4, 128)[0].backward(bq_g)

    ball_fwd_bwd()
    torch.cuda.synchronize()
    t_bf = timer.time(ball_fwd, reps)
    t_bfb = timer.time(ball_fwd_bwd, reps)
    propagation = {
        "three_nn": {"ms": t_tn * 1e3, "tops": PAIR_OPS * B * N * C2_NPOINT / t_tn / 1e12},
        "three_interpolate": {"ms": t_ti * 1e3, "gbps": interp_bytes / t_ti / 1e9},
        "three_interpolate_fwd_bwd": {"ms": t_tib * 1e3, "gbps": 2 * interp_bytes / t_tib / 1e9},
        "query_and_group_C64_S32": {"ms": t_gf * 1e3, "gbps": group_bytes / t_gf / 1e9},
        "query_and_group_fwd_bwd": {"ms": t_gfb * 1e3},
        "QueryAndGroup_layer_ball_query_plus_group": {"ms": t_gl * 1e3},
        "ball_query_r04_K128_fwd": {"ms": t_bf * 1e3},
        "ball_query_r04_K128_fwd_bwd": {"ms": t_bfb * 1e3},
    }

    overlapped = pipelined_steps(mp, xyz, args.steps, args.warmup)

    kernel = fps_kernel_name(N)
    achieved = fps_ops / t_fps
    # One workgroup per cloud: B of the 256 CUs run the FPS kernel.
    occupied = min(B, MI355X_CUS) * MI355X_VALU_ISSUE_PER_CU
    traffic = profiled_traffic(kernel, "c2")
    result = {
        "metric": "points/sec for FPS+ball_query+kNN at B=32,N=4096; % of HBM/FP32 roofline",
        "value": B * N / wall,
        "unit": "points/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (BASELINE.json config 2 generator, seed 2)",
        "config": {
            "workload": "c2 PointNet++ MSG layer: B=32 N=4096 FPS1024 + ball(0.1,16)(0.2,32)"
                        "(0.4,128) + kNN16",
            "B": B, "N": N, "npoint": C2_NPOINT,
        },
        "ops": {"fps": op(t_fps, fps_ops), "ball_query_x3": op(t_ball, ball_ops),
                "knn": op(t_knn, knn_ops)},
        "ball_query_x3_one_scan_not_in_value": {
            "what": "mps_pointops.ball_query_multi: the 3 radii over all 1024 centres in one "
                    "scan (each pair's distance computed once), the same outputs bit for bit",
            **op(t_ball_multi, ball_ops),
        },
        "step": "mps_pointops.fps_ball_knn: FPS, centre gather, 3 ball queries and kNN of one "
                f"batch, the ball queries of each {C2_CHUNK}-centre chunk (all 3 radii in one scan) "
                "overlapped with the rest of FPS, kNN once after the last chunk",
        "sequential_not_in_value": {
            "what": "the same batch as separate calls on one stream (FPS, then the ball queries "
                    "and kNN on centres gathered beforehand, outside the timed region)",
            "ms_per_step": wall_sequential * 1e3,
            "points_per_s": B * N / wall_sequential,
        },
        "sum_of_ops_not_in_value": {
            "what": "B*N / (t_FPS + sum of the 3 ball-query times + t_kNN), each the kernel time "
                    "of its separate call (HIP events on the launch stream)",
            "ms": (t_fps + t_ball + t_knn) * 1e3,
            "points_per_s": B * N / (t_fps + t_ball + t_knn),
        },
        "propagation_not_in_value": propagation,
        "two_streams_not_in_value": {
            "what": "the same K steps software-pipelined over two default-priority streams: "
                    "FPS of batch i+1 runs beside the ball queries and kNN of batch i, which "
                    "use batch i's FPS output (FPS occupies 32 of the 256 CUs)",
            "ms_per_step": overlapped * 1e3,
            "points_per_s": B * N / overlapped,
        },
        "roofline": {
            "kernel": kernel,
            "bound": "valu",
            "compute": "fp32 VALU, unfused (no MFMA, no FMA, no packed fp32)",
            "achieved": achieved / 1e12,
            "peak": MI355X_FP32_PEAK / 1e12,
            "unit": "TFLOP/s",
            "frac": achieved / MI355X_FP32_PEAK,
            "traffic": traffic,
            "valu_issue_peak": MI355X_VALU_ISSUE / 1e12,
            "frac_valu_issue": achieved / MI355X_VALU_ISSUE,
            "occupied_cus": min(B, MI355X_CUS),
            "frac_occupied_cu_issue": achieved / occupied,
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(xyz_cpu, args.cpu_clouds, args.cpu_warmup,
                                              args.cpu_repeats)
    return result


def run_other(args) -> dict:
    """The other BASELINE.json configurations (kernel time on the launch
    stream, inputs resident in HBM).  Reported for the record; the headline
    metric is config 2."""
    import mps_pointops as mp

    dev = torch.device("cuda", 0)
    stream_timer = KernelTimer(torch.cuda.current_stream(dev))
    reps = max(3, args.steps)

    class Warm:
        """Runs `warmup` untimed calls (first-use library loading, caches)
        before the event-timed ones."""

        @staticmethod
        def time(fn, n):
            for _ in range(max(1, args.warmup)):
                fn()
            torch.cuda.synchronize()
            return stream_timer.time(fn, n)

    timer = Warm()
    out = {"n_gpus": 1, "dtype": "f32", "data": f"synthetic (BASELINE.json {args.config} generator)",
           "higher_is_better": True, "vs_baseline": None}
    if args.config == "c1":
        x = make_c1().to(dev)
        B, N, _ = x.shape
        idx = mp.furthest_point_sample(x, 512)
        c = x.gather(1, idx[..., None].expand(-1, -1, 3)).contiguous()
        t_fps = timer.time(lambda: mp.furthest_point_sample(x, 512), reps)
        t_ball = timer.time(lambda: mp.ball_query(c, x, 0.2, 32), reps)
        t_knn = timer.time(lambda: mp.knn(c, x, 16), reps)
        t = t_fps + t_ball + t_knn
        out.update(metric="points/sec for FPS512+ball(0.2,32)+kNN16 at B=16,N=1024", value=B * N / t,
                   unit="points/s", config={"workload": "c1 PointNet++ SSG grouping B=16 N=1024"},
                   ops_ms={"fps": t_fps * 1e3, "ball_query": t_ball * 1e3, "knn": t_knn * 1e3})
    elif args.config == "c3":
        x = make_c3().to(dev)
        N = x.shape[1]
        idx = mp.furthest_point_sample(x, 16384)
        c = x.gather(1, idx[..., None].expand(-1, -1, 3)).contiguous()
        r = max(1, reps // 5)
        t_fps = timer.time(lambda: mp.furthest_point_sample(x, 16384), r)
        t_ball = timer.time(lambda: mp.ball_query(c, x, 0.5, 32), r)
        fps_ops = FPS_OPS_PER_POINT_STEP * 16384 * N
        ball_ops = PAIR_OPS * ball_scanned_pairs(mp.ball_query(c, x, 0.5, 32)[1], N)
        # Beside the metric: the same slab generator at 4x the points, which
        # takes the streaming kernel (above 2^21 points).
        x4 = make_c3(N=1 << 22).to(dev)
        t_fps4 = timer.time(lambda: mp.furthest_point_sample(x4, 16384), r)
        out.update(metric="points/sec for FPS16384+ball(0.5,32) at B=1,N=1048576",
                   value=N / (t_fps + t_ball), unit="points/s",
                   config={"workload": "c3 large single-cloud FPS (LiDAR-like slab) + ball query"},
                   ops_ms={"fps": t_fps * 1e3, "ball_query": t_ball * 1e3,
                           "fps_4194304_points_streaming": t_fps4 * 1e3},
                   tops={"fps": fps_ops / t_fps / 1e12, "ball_query": ball_ops / t_ball / 1e12,
                         "fps_4194304_points_streaming":
                             FPS_OPS_PER_POINT_STEP * 16384 * (1 << 22) / t_fps4 / 1e12})
    elif args.config == "c4":
        from mps_pointops import _native

        ref, query, feat = (t.to(dev) for t in make_c4())
        r = max(1, reps // 5)
        t_knn = timer.time(lambda: mp.knn(query, ref, 16), r)
        t_feat = timer.time(lambda: mp.knn(feat, feat, 20), reps)
        # DGCNN's deeper EdgeConv width (D=128) at the same sizes, and the
        # reference's own feature-kNN sizes (Q = N = 1024, k = 20, D = 64/128).
        g = torch.Generator().manual_seed(44)
        feat128 = torch.randn(8, 2048, 128, generator=g).to(dev)
        small = {d: torch.randn(1, 1024, d, generator=g).to(dev) for d in (64, 128)}
        t_feat128 = timer.time(lambda: mp.knn(feat128, feat128, 20), reps)
        t_small = {d: timer.time(lambda x=x: mp.knn(x, x, 20), reps) for d, x in small.items()}
        M, N = query.shape[1], ref.shape[1]
        Bf, Nf, D = feat.shape
        # The same sizes on clustered references with uniform queries, through
        # the public call (grid search, far queries left to the linear pass)
        # and through the brute-force kernel alone, for comparison.
        cref, cquery = (t.to(dev) for t in make_c4_clustered())
        t_clustered = timer.time(lambda: mp.knn(cquery, cref, 16), r)
        bd = torch.empty(1, M, 16, device=dev)
        bi = torch.empty(1, M, 16, dtype=torch.long, device=dev)
        t_brute = timer.time(lambda: _native.call(
            "pointops_knn3", cquery.data_ptr(), cref.data_ptr(), bd.data_ptr(), bi.data_ptr(),
            1, M, N, 16, _native.stream(dev)), 1)
        out.update(metric="queries/sec for exact kNN16, 131072 queries x 1048576 refs",
                   value=M / t_knn, unit="queries/s",
                   config={"workload": "c4 kNN at scale + DGCNN feature kNN (8,2048,64) K=20"},
                   ops_ms={"knn": t_knn * 1e3, "dgcnn_feature_knn": t_feat * 1e3,
                           "dgcnn_feature_knn_d128": t_feat128 * 1e3,
                           "feature_knn_q1024_d64": t_small[64] * 1e3,
                           "feature_knn_q1024_d128": t_small[128] * 1e3,
                           "knn_clustered_uniform_queries": t_clustered * 1e3,
                           "knn_clustered_brute_force_kernel": t_brute * 1e3},
                   knn_path="grid search (knn_grid.hip): examines the cells around each query, "
                            "not all M x N pairs",
                   tops={"knn_brute_force_equivalent": PAIR_OPS * M * N / t_knn / 1e12,
                         "dgcnn_feature_knn": (3 * D - 1) * Bf * Nf * Nf / t_feat / 1e12,
                         "dgcnn_feature_knn_d128": (3 * 128 - 1) * Bf * Nf * Nf / t_feat128 / 1e12})
    elif args.config == "c5":
        y1, y2 = (t.to(dev) for t in make_c5())
        B, P, _ = y1.shape
        a = y1.clone().requires_grad_()
        b = y2.clone().requires_grad_()

        def fwd_bwd():
            loss, _ = mp.chamfer_distance(a, b)
            loss.backward()

        t = timer.time(fwd_bwd, reps)
        out.update(metric="points/sec for squared-L2 Chamfer forward+backward at B=32,P=8192",
                   value=2 * B * P / t, unit="points/s",
                   config={"workload": "c5 Chamfer mean/mean fwd+bwd, both directions"},
                   ops_ms={"chamfer_fwd_bwd": t * 1e3},
                   tops={"forward_pairs": 2 * PAIR_OPS * B * P * P / t / 1e12})
    return out


def probe() -> None:
    """One pass of each config-2 kernel (the metric's FPS, ball queries --
    separately and in one multi-radius scan -- and kNN, then three_nn and three_interpolate forward and backward of C=128
    features, and the set-abstraction layer: the pointnet2-form ball query
    (0.2, 32) and the grouping of C=64 features forward and backward) plus a
    256 MiB device copy, three times, for hardware-counter runs (the copy's
    FETCH_SIZE/WRITE_SIZE give the scale of the counters against known
    bytes)."""
    import mps_pointops as mp
    from mps_pointops import group as grouping

    xyz = make_c2().cuda()
    B, N, _ = xyz.shape
    g = torch.Generator().manual_seed(9)
    feats = torch.randn(B, 128, C2_NPOINT, generator=g).cuda().requires_grad_()
    upstream = torch.randn(B, 128, N, generator=g).cuda()
    sa_feats = torch.randn(B, 64, N, generator=g).cuda().requires_grad_()
    sa_up = torch.randn(B, 67, C2_NPOINT, 32, generator=g).cuda()
    sa_layer = grouping.QueryAndGroup(0.2, 32)
    src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        idx = mp.furthest_point_sample(xyz, C2_NPOINT)
        centres = xyz.gather(1, idx[..., None].expand(-1, -1, 3)).contiguous()
        for radius, k in C2_RADII:
            mp.ball_query(centres, xyz, radius, k)
        mp.ball_query_multi(centres, xyz, [r for r, _ in C2_RADII], [k for _, k in C2_RADII])
        mp.knn(centres, xyz, C2_KNN_K)
        tn_d, tn_i = mp.three_nn(xyz, centres)
        inv = 1.0 / (tn_d + 1e-8)
        w = (inv / inv.sum(-1, keepdim=True)).contiguous()
        feats.grad = None
        mp.three_interpolate(feats, tn_i, w).backward(upstream)
        sa_feats.grad = None
        sa_layer(xyz, centres, sa_feats).backward(sa_up)
        dst.copy_(src)
    torch.cuda.synchronize()
    print("probe: 3 x (fps, 3 ball queries, their one-scan form, knn, three_nn, three_interpolate fwd+bwd, "
          "QueryAndGroup fwd+bwd, 256 MiB copy) done", flush=True)


def pipeline_trace(calls: int = 20) -> None:
    """The timed step alone (mps_pointops.fps_ball_knn at config 2, chunk
    C2_CHUNK, as the benchmark times it) `calls` times after two warm-up calls,
    for a kernel trace of the overlapped front end."""
    import mps_pointops as mp

    xyz = make_c2().cuda()
    radii = [r for r, _ in C2_RADII]
    ks = [k for _, k in C2_RADII]
    for _ in range(2 + calls):
        mp.fps_ball_knn(xyz, C2_NPOINT, radii, ks, C2_KNN_K, chunk=C2_CHUNK)
    torch.cuda.synchronize()
    print(f"pipeline: {2 + calls} x fps_ball_knn (chunk {C2_CHUNK}) done", flush=True)


def main() -> None:
    parser = argparse.ArgumentParser()
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=3)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--cpu-clouds", type=int, default=32)
    parser.add_argument("--cpu-warmup", type=int, default=3)
    parser.add_argument("--cpu-repeats", type=int, default=20)
    parser.add_argument("--config", default="c2", choices=["c1", "c2", "c3", "c4", "c5"],
                        help="workload; the headline metric (and the default) is c2")
    parser.add_argument("--pipeline-trace", action="store_true",
                        help=f"run only the timed step (fps_ball_knn, chunk {C2_CHUNK}) 22 times, "
                             "for a kernel trace")
    parser.add_argument("--probe", action="store_true",
                        help="run each config-2 kernel 3 times (for rocprofv3 counter passes)")
    args = parser.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one MI355X; every workload here runs on one "
                          "GPU (sharding the batch of clouds across GPUs is a design, not built)",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    if args.probe:
        probe()
        return
    if args.pipeline_trace:
        pipeline_trace()
        return
    result = run(args) if args.config == "c2" else run_other(args)
    if args.config != "c2" and not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline_other(args.config)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
