"""Benchmark of the spira_amd hot path on one MI355X.

Headline (BASELINE.json metric): end-to-end latency of the config-4 workload
-- SparseResUNet42, fp16, random-init weights, on a 200k-voxel synthetic
indoor scene -- timed like the reference (scripts/end_to_end_experiment.py:
156-252): kernel-map cache reset, then `order()` (pack + sort), the
network-wide kernel-map build (`add_all_kernel_maps`) and the forward pass
inside one event-timed region.  Also reported on the same run:
  * kmap_build_us: one kernel-map search (config 2, ~100k LiDAR voxels,
    k=3, 64-bit keys, output-stationary layout) as in mapping_experiment.py;
  * layer_ms: one output-stationary fp16 layer (config 3, C=64);
  * config5_ms: the large-kernel network of config 5 (SparseResNetLarge, k=5,
    fp16) end to end on the ~300k-voxel LiDAR-plus-blobs scene, timed like
    the headline (10 steps after 5 warm-ups);
  * roofline: the dominant kernel (output-stationary MFMA conv) against its
    binding roofline -- HBM for the full-resolution 96->96 layer, whose
    algorithmic bytes take longer at peak bandwidth than its flops at peak
    MFMA rate (the MFMA fraction is reported beside it) -- and
    kmap_roofline: the map search against HBM peak;
  * cpu_baseline: the same end-to-end pipeline run by the OpenMP CPU
    restatement (oracle/) on the host cores (one scene).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
# HBM bytes per launch of the dominant kernel (os_kernel<3,0,true,8,false,1>, 200k
# voxels, 96 -> 96): rocprofv3 --pmc FETCH_SIZE and --pmc WRITE_SIZE over
# `bench.py --no-cpu --only layer,calib`, each scaled by what the counter
# reads for the calibration leg's 256 MiB copy (FETCH_SIZE x 2.000,
# WRITE_SIZE x 1.000): 68049 KiB fetched, 37578 KiB written.
DOMINANT_TRAFFIC_BYTES = 68049 * 1024 * 2.0 + 37578 * 1024 * 1.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--dataflow", type=int, default=0, help="map dataflow used by every layer")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-fuse", action="store_true", help="run batch norm / ReLU / residual adds unfused")
    p.add_argument("--only", default="", help="comma list of legs: e2e,kmap,layer,config5 (calib: a plain 256 MiB "
                                              "device copy, the reference point of the HBM byte counters)")
    return p.parse_args()


class Timer:
    """HIP-event timing on the current stream (the one the kernels run on)."""

    def __init__(self, torch):
        self.torch = torch

    def __call__(self, fn, reps: int, warmup: int = 2):
        torch = self.torch
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        times = []
        for _ in range(reps):
            s.record()
            fn()
            e.record()
            e.synchronize()
            times.append(s.elapsed_time(e))
        return float(np.mean(times)), float(np.min(times))


def e2e_leg(torch, args, coords_np, net="UNet", steps=None, warmup=None):
    """End-to-end step of `net` (UNet: SparseResUNet42, config 4; ResNetLarge:
    the k = 5 SparseResNetLarge, config 5): map cache reset, order(), the
    network-wide map build and the forward pass, event-timed."""
    import spira_amd
    from spira_amd.networks import SparseResNetLarge, SparseResUNet42, kmap_schedule
    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    cin = 3 if net == "UNet" else 4
    model = (SparseResUNet42 if net == "UNet" else SparseResNetLarge)(in_channels=cin).to(dev).half().eval()
    steps = args.steps if steps is None else steps
    warmup = args.warmup if warmup is None else warmup
    if not args.no_fuse:
        spira_amd.nn.fuse_epilogues(model)
    cache = spira_amd.nn.KernelMapCache()
    spira_amd.set_kernel_map_cache(model, cache)
    for m in model.modules():
        if isinstance(m, spira_amd.nn.SparseConv):
            m._tunable_config["map_dataflow"] = args.dataflow
    ts, ks, ss = kmap_schedule(net)
    coords = torch.from_numpy(coords_np).to(dev)
    feats = torch.randn(coords.shape[0], cin, device=dev, dtype=torch.float16)

    def step():
        cache.reset()
        x = spira_amd.SparseTensor(coordinates=coords, features=feats, double=True)
        x.order()
        cache.add_all_kernel_maps(x._coordinates, ks, ss, ts, (1, 1, 1), [args.dataflow] * len(ks))
        return model(x)

    with torch.no_grad():
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        s.record()
        for _ in range(steps):
            out = step()
        e.record()
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) * 1e3 / steps
        ms = s.elapsed_time(e) / steps
    return ms, wall, model, [o._features for o in out]


def kmap_leg(torch, keys_np):
    """Config 2: build_kmap(dataflow=0) per call as the reference times it
    (HIP events around the Python call, host overhead included) and the
    search kernel alone (back-to-back launches from C++)."""
    from spira_amd.nn import functional as F
    from spira_amd.nn.functional import _native
    dev = torch.device("cuda:0")
    keys = torch.from_numpy(keys_np).to(dev)
    timer = Timer(torch)
    S = T = keys.shape[0]
    out = {}
    for k in (3, 5):
        mean_ms, min_ms = timer(lambda: F.build_kmap(keys, keys, k, 1, 0), reps=20, warmup=3)
        kern_ms = _native._C.time_kmap_search(keys, keys, (k, k, k), (1, 1, 1), 50)
        K = k ** 3
        nbytes = 8 * S + 8 * T + 4 * K * T
        out[k] = {"us": mean_ms * 1e3, "min_us": min_ms * 1e3, "kernel_us": kern_ms * 1e3, "bytes": nbytes,
                  "gbs": nbytes / (kern_ms * 1e-3) / 1e9}
    return out


def layer_leg(torch, keys_np, channels=(16, 32, 64, 128, 256), reps=20):
    """Config 3 (LiDAR, k=3, s=1): the output-stationary fp16 layer per
    channel count, kernel only (back-to-back launches from C++)."""
    from spira_amd.nn import functional as F
    from spira_amd.nn.functional import _native
    dev = torch.device("cuda:0")
    keys = torch.from_numpy(keys_np).to(dev)
    m = F.build_kmap(keys, keys, 3, 1, 0)
    S = T = keys.shape[0]
    P = int((m[2][:T] >= 0).sum().item())
    out = {}
    for C in channels:
        X = torch.randn(S, C, device=dev, dtype=torch.float16)
        W = (torch.randn(27, C, C, device=dev) / np.sqrt(27 * C)).half()
        ms = _native._C.time_conv_os(S, T, m[2], X, W, reps)
        flops = 2.0 * P * C * C
        out[C] = {"ms": ms, "tflops": flops / (ms * 1e-3) / 1e12, "flops": flops}
    return {"pairs": P, "voxels": S, "per_C": out}


def dominant_leg(torch, keys_np, C=96, reps=20):
    """The dominant kernel of the config-4 run: the output-stationary fp16
    layer at full resolution (200k indoor voxels, k=3, 96 -> 96 channels),
    kernel only."""
    from spira_amd.nn import functional as F
    from spira_amd.nn.functional import _native
    dev = torch.device("cuda:0")
    keys = torch.from_numpy(keys_np).to(dev)
    m = F.build_kmap(keys, keys, 3, 1, 0)
    S = T = keys.shape[0]
    P = int((m[2][:T] >= 0).sum().item())
    X = torch.randn(S, C, device=dev, dtype=torch.float16)
    W = (torch.randn(27, C, C, device=dev) / np.sqrt(27 * C)).half()
    ms = _native._C.time_conv_os(S, T, m[2], X, W, reps)
    flops = 2.0 * P * C * C
    # algorithmic bytes: fp16 features read and written once, fp16 weights,
    # the int32 map read once
    nbytes = 2.0 * (S * C + T * C) + 2.0 * 27 * C * C + 4.0 * 27 * T
    return {"ms": ms, "flops": flops, "tflops": flops / (ms * 1e-3) / 1e12, "pairs": P, "C": C,
            "bytes": nbytes, "gbs": nbytes / (ms * 1e-3) / 1e9}


def calib_leg(torch, mib=256, reps=5):
    """A plain device-to-device copy of a known size: reads and writes
    `mib` MiB per launch.  Run under rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE
    it gives the factor that turns those counters into bytes."""
    dev = torch.device("cuda:0")
    x = torch.empty(mib * (1 << 20) // 2, dtype=torch.float16, device=dev).uniform_()
    y = torch.empty_like(x)
    for _ in range(reps):
        y.copy_(x)
    torch.cuda.synchronize()
    return {"bytes_each_way": mib * (1 << 20), "reps": reps}


# ---------------------------------------------------------------------------
# CPU baseline: the same end-to-end pipeline on the host through the oracle
# ---------------------------------------------------------------------------
def cpu_e2e(model, coords_np, feats_np):
    """The same network end to end on the host through the oracle (fp32,
    OpenMP C restatement of the maps and convolutions)."""
    from oracle.network import network_forward
    return network_forward(model, coords_np, feats_np)


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: every GPU box here has one MI355X; "
                                   "use --gpus 1"}))
        sys.exit(2)
    import torch
    from spira_amd import scenes

    legs = set(args.only.split(",")) if args.only else {"e2e", "kmap", "layer", "config5"}
    with open(os.path.join(ROOT, "BASELINE.json")) as f:
        baseline = json.load(f)

    indoor = scenes.indoor()
    res = {"metric": baseline["metric"], "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
           "data": "synthetic (seeded scenes, random-init weights)"}
    cfg = {"workload": "config4: SparseResUNet42 fp16, 200k-voxel indoor scene, end-to-end "
                       "(order + network-wide kernel maps + forward)",
           "voxels": int(indoor.shape[0]), "key_bits": 64, "map_dataflow": args.dataflow}
    model = None
    if "e2e" in legs:
        ms, wall, model, _ = e2e_leg(torch, args, indoor)
        res["value"] = ms
        res["ms_per_step"] = ms
        res["wall_ms_per_step"] = wall
    if "config5" in legs:
        # config 5: the large-kernel (k = 5) SparseResNetLarge on the ~300k-voxel
        # scene of merged LiDAR rings and Gaussian blobs, timed like config 4
        blobs = scenes.lidar_blobs()
        c5, _, _, _ = e2e_leg(torch, args, blobs, net="ResNetLarge", steps=10, warmup=5)
        res["config5_ms"] = c5
        cfg["config5_voxels"] = int(blobs.shape[0])
    lidar = scenes.lidar()
    from oracle import oracle as orc
    lkeys, _ = orc.flatten_sort(lidar, True)
    if "kmap" in legs:
        km = kmap_leg(torch, lkeys)
        res["kmap_build_us"] = km[3]["us"]
        res["kmap_build_us_k5"] = km[5]["us"]
        res["kmap_kernel_us"] = km[3]["kernel_us"]
        res["kmap_kernel_us_k5"] = km[5]["kernel_us"]
        res["kmap_roofline"] = {"bound": "hbm", "achieved": km[3]["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                "frac": km[3]["gbs"] / HBM_PEAK_GBS, "traffic": None,
                                "kernel": "kmap_search_kernel<u64,3> (config 2, k=3, OS layout)",
                                "algorithmic_bytes": km[3]["bytes"]}
        res["kmap_roofline_k5"] = {"achieved": km[5]["gbs"], "frac": km[5]["gbs"] / HBM_PEAK_GBS,
                                   "algorithmic_bytes": km[5]["bytes"]}
        cfg["kmap_voxels"] = int(lkeys.shape[0])
    if "layer" in legs:
        ly = layer_leg(torch, lkeys)
        res["layer_ms"] = ly["per_C"][64]["ms"]
        res["layer_sweep"] = {str(c): {"ms": v["ms"], "tflops": v["tflops"],
                                       "frac": v["tflops"] / MFMA_F16_PEAK_TFLOPS}
                              for c, v in ly["per_C"].items()}
        res["layer_pairs"] = ly["pairs"]
        ikeys, _ = orc.flatten_sort(indoor, True)
        dm = dominant_leg(torch, ikeys)
        # the binding roofline: the larger of bytes / HBM peak and flops /
        # MFMA peak
        hbm_bound = dm["bytes"] / (HBM_PEAK_GBS * 1e9) >= dm["flops"] / (MFMA_F16_PEAK_TFLOPS * 1e12)
        if hbm_bound:
            rl = {"bound": "hbm", "achieved": dm["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                  "frac": dm["gbs"] / HBM_PEAK_GBS}
        else:
            rl = {"bound": "mfma", "achieved": dm["tflops"], "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                  "frac": dm["tflops"] / MFMA_F16_PEAK_TFLOPS}
        res["roofline"] = {**rl, "mfma_tflops": dm["tflops"], "mfma_frac": dm["tflops"] / MFMA_F16_PEAK_TFLOPS,
                           "algorithmic_bytes": dm["bytes"],
                           "traffic": DOMINANT_TRAFFIC_BYTES,
                           "traffic_gbs": DOMINANT_TRAFFIC_BYTES / (dm["ms"] * 1e-3) / 1e9,
                           "kernel": "os_kernel<3,0,true,8,false,1> (config 4 full resolution, 200k voxels, k=3, 96->96, "
                                     "fp16, 128-channel steps)",
                           "ms": dm["ms"], "algorithmic_flops": dm["flops"], "valid_pairs": dm["pairs"]}
    if "calib" in legs:
        res["calib"] = calib_leg(torch)
    if not args.no_cpu and model is not None:
        feats = np.random.default_rng(0).standard_normal((indoor.shape[0], 3)).astype(np.float32)
        t0 = time.perf_counter()
        cpu_e2e(model, indoor, feats)
        cpu_ms = (time.perf_counter() - t0) * 1e3
        res["cpu_baseline"] = {"value": cpu_ms, "unit": "ms", "cores": orc.threads(), "kind": "port",
                               "sample": "one full config-4 scene end-to-end (sort, downsample, all maps, "
                                         "all 42 layers, fp32) by the OpenMP oracle"}
    res["config"] = cfg
    print(json.dumps(res))


if __name__ == "__main__":
    main()
