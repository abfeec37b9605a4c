"""Benchmark of the spira_amd hot path on one MI355X.

Headline (BASELINE.json metric): end-to-end latency of the config-4 workload
-- SparseResUNet42, fp16, random-init weights, on a 200k-voxel synthetic
indoor scene -- timed like the reference (scripts/end_to_end_experiment.py:
126-252): the selector (spira_amd.tune) runs first, outside the timed region;
then per step the kernel-map cache is reset and `order()` (pack + sort), the
network-wide kernel-map build (`add_all_kernel_maps`) and the forward pass
run inside one event-timed region.  Also reported on the same run:
  * config 4 per layer (in-network): every convolution's time inside one
    steady-state step (HIP events at layer boundaries), its algorithmic bytes
    and flops, and the per-step dominant family (stride, C_in, C_out,
    offsets) with its binding roofline -> `roofline`;
  * config5_ms: the large-kernel SparseResNetLarge (k = 5, fp16) end to end
    on the ~300k-voxel LiDAR-plus-blobs scene, timed like the headline;
  * kmap: the map search of config 2 (~100k LiDAR voxels, 64-bit keys) for
    k = 3 / 5 at stride 1 / 2, per API call (as mapping_experiment.py:81-101
    times it) and kernel only, against HBM peak;
  * layers: config 3 (LiDAR, k = 3, stride 1, C = 16 ... 256), every
    dataflow (output-stationary, fused weight-stationary, gather-GEMM-scatter,
    hybrids 3-8) timed per layer call (layerwise_experiment.py:100-186), the
    selector's pick (the fastest), and each against the fp16 MFMA peak;
  * config1_fp32: config 1's fp32 layer (20k voxels, k = 3, C = 32; also
    C = 64, 128) on the fp32 MFMA kernel, per call and kernel only, against
    the fp32 matrix peak;
  * cpu_baseline: the same legs by the OpenMP CPU restatement (oracle/) on
    the host cores, each checked against the GPU result: config 4 end to end
    (headline), the config-2 k = 3 map and a config-3 C = 64 layer.
Opt-in legs for counter passes (--only): family (config 4's families, each
layer alone at its tuned launch), c5family (config 5's 125-offset layer
shapes alone) and calib (a plain 256 MiB copy, the HBM counters' reference).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--only legs]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from collections import defaultdict

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
MFMA_F32_PEAK_TFLOPS = 157.3
# HBM bytes per launch of each submanifold family's output-stationary kernel
# (plus the finalize kernel of a launch with offset splits), at the tuned
# launch the selector chose in the measured run: the family leg replays every
# family 20 times back to back, and the counters are averaged over those
# dispatches.  From rocprofv3 --pmc FETCH_SIZE and --pmc WRITE_SIZE over
# `bench.py --only e2e,family,calib --no-cpu --tune-dir D --steps 2
# --warmup 1`, each scaled by what the counter reads for the calibration
# leg's 256 MiB copy (FETCH_SIZE x 2.000, WRITE_SIZE x 1.000).  The
# commands, tunings and raw figures are in profiles/os_kernel_traffic.md; a
# default run re-tunes and can choose other launches, whose traffic differs.
MEASURED_TRAFFIC = {
    "s1 3->32 K27": 59147816,  # FETCH 22529.4 KiB, WRITE 12707.2 KiB
    "s1 32->32 K27": 82594203,  # FETCH 33973.9 KiB, WRITE 12717.2 KiB
    "s1 96->96 K27": 177703176,  # FETCH 67987.5 KiB, WRITE 37576.5 KiB
    "s1 128->96 K27": 188732655,  # FETCH 73375.5 KiB, WRITE 37572.4 KiB
    "s2 32->32 K27": 93550079,  # FETCH 40831.6 KiB, WRITE 9702.2 KiB
    "s2 96->96 K27": 230775517,  # FETCH 98282.5 KiB, WRITE 28820.8 KiB
    "s2 128->96 K27": 252398889,  # FETCH 108841.0 KiB, WRITE 28822.3 KiB
    "s4 32->64 K27": 40333856,  # FETCH 15465.3 KiB, WRITE 8460.9 KiB
    "s4 64->64 K27": 56965110,  # FETCH 23586.8 KiB, WRITE 8460.9 KiB
    "s4 128->128 K27": 133386743,  # FETCH 56674.9 KiB, WRITE 16921.8 KiB
    "s4 192->128 K27": 175078752,  # FETCH 77034.3 KiB, WRITE 16921.8 KiB
    "s8 64->128 K27": 13367064,  # FETCH 4396.8 KiB, WRITE 4261.0 KiB
    "s8 128->128 K27": 20248062,  # FETCH 7757.0 KiB, WRITE 4261.0 KiB
    "s8 256->256 K27": 50210735,  # FETCH 20234.5 KiB, WRITE 8568.8 KiB
    "s8 384->256 K27": 98760791,  # FETCH 43955.8 KiB, WRITE 8542.9 KiB
    "s16 128->256 K27": 19567968,  # FETCH 8556.5 KiB, WRITE 1998.0 KiB
    "s16 256->256 K27": 61090076,  # FETCH 18842.0 KiB, WRITE 21978.0 KiB
}
# the same for the config-2 k=3 stride-1 map search (`--only kmap,calib`)
KMAP_TRAFFIC = 16050790  # FETCH 2558.8 KiB, WRITE 10557.0 KiB


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--dataflow", type=int, default=0, help="map dataflow of every layer without the selector")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    p.add_argument("--tune-dir", default=None,
                   help="keep the selector's result in this folder and reuse it when present "
                        "(profiler passes replay one selection instead of searching under the counters)")
    p.add_argument("--no-fuse", action="store_true", help="run batch norm / ReLU / residual adds unfused")
    p.add_argument("--no-tune", action="store_true", help="skip the selector (library default launch choices)")
    p.add_argument("--only", default="", help="comma list of legs: e2e, config5, kmap, layer, family (the "
                                              "dominant family's layers alone, for counters), c5family (config 5's "
                                              "125-offset layer shapes alone, for counters), calib (a plain "
                                              "256 MiB device copy: the reference point of the HBM counters)")
    p.add_argument("--concurrent-maps", action="store_true",
                   help="build every layer map on a side stream of its own (the library's opt-in fan-out)")
    p.add_argument("--layer-table", default="", help="write the per-layer in-network table (markdown) here")
    return p.parse_args()


def event_time(torch, fn, reps: int, warmup: int = 2) -> float:
    """Mean ms per call of fn() between HIP events on the current stream."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) / reps


# ---------------------------------------------------------------------------
# end to end (configs 4 and 5)
# ---------------------------------------------------------------------------
def e2e_inputs(torch, coords_np, cin, seed=7):
    """Coordinates and fp16 N(0, 1) features of an end-to-end run, on the GPU
    (seeded, so that the CPU baseline sees the same features)."""
    g = torch.Generator().manual_seed(seed)
    feats = torch.randn(coords_np.shape[0], cin, generator=g).half()
    dev = torch.device("cuda:0")
    return torch.from_numpy(coords_np).to(dev), feats.to(dev)


def layer_groups(net):
    """(source stride, kernel size, layer stride) of each network-wide map,
    the key under which the selector reports a map's dataflow (the
    reference's lookup, scripts/end_to_end_experiment.py:141-150)."""
    from spira_amd.networks import kmap_schedule
    _, ks, ss = kmap_schedule(net)
    return [(tuple(ss[i]), tuple(ks[i]), tuple(b // a for a, b in zip(ss[i], ss[i + 1]))) for i in range(len(ks))]


class E2E:
    """One end-to-end workload: model, inputs, map schedule, and the step
    (cache reset, order(), network-wide map build, forward)."""

    def __init__(self, torch, args, coords_np, net):
        import spira_amd
        from spira_amd.networks import SparseResNetLarge, SparseResUNet42, kmap_schedule
        self.torch, self.net = torch, net
        dev = torch.device("cuda:0")
        torch.manual_seed(0)
        self.cin = 3 if net == "UNet" else 4
        self.model = (SparseResUNet42 if net == "UNet" else SparseResNetLarge)(in_channels=self.cin)
        self.model = self.model.to(dev).half().eval()
        if not args.no_fuse:
            spira_amd.nn.fuse_epilogues(self.model)
        self.cache = spira_amd.nn.KernelMapCache()
        spira_amd.set_kernel_map_cache(self.model, self.cache)
        for m in self.model.modules():
            if isinstance(m, spira_amd.nn.SparseConv):
                m._tunable_config["map_dataflow"] = args.dataflow
        self.ts, self.ks, self.ss = kmap_schedule(net)
        self.coords, self.feats = e2e_inputs(torch, coords_np, self.cin)
        self.dataflows = [args.dataflow] * len(self.ks)
        self.chosen = None
        self.tune_dir = args.tune_dir
        self.randomise_norms()

    def randomise_norms(self, seed=42):
        """Batch-norm statistics and affine parameters drawn at random (the
        parity tests' choice): with the library's default statistics the
        random-init network shrinks its activations ~3x per layer, into
        fp16's subnormal range at the coarse levels."""
        import spira_amd
        g = self.torch.Generator().manual_seed(seed)
        for m in self.model.modules():
            if isinstance(m, spira_amd.nn.BatchNorm):
                n = m.running_mean.numel()
                m.running_mean.copy_(0.1 * self.torch.randn(n, generator=g))
                m.running_var.copy_(0.5 + self.torch.rand(n, generator=g))
                m.weight.data.copy_(0.5 + self.torch.rand(n, generator=g))
                m.bias.data.copy_(0.1 * self.torch.randn(n, generator=g))

    def tune(self):
        """The selector: dataflow per layer group (0-2, as fast as the model
        runs them), then the output-stationary launch choices per layer and
        the row order per map."""
        import tempfile
        import spira_amd

        def sample():
            x = spira_amd.SparseTensor(coordinates=self.coords, features=self.feats, double=True)
            return x.order()

        with tempfile.TemporaryDirectory() as tmp:
            d = self.tune_dir or tmp
            self.model, groups = spira_amd.tune(self.model, [sample() for _ in range(11)], self.cache,
                                                map_dataflow_options=[0, 1, 2], test_force_os=False, n_samples=10,
                                                save_dir=d, tune_tag=self.net, force_retune=self.tune_dir is None,
                                                allow_gs_tuning=False, return_dataflows=True)
        self.dataflows = [groups.get(g, d) for g, d in zip(layer_groups(self.net), self.dataflows)]
        self.chosen = {"map_dataflows": self.dataflows,
                       "row_orders": {str(k): v for k, v in self.cache.row_order_requests.items()}}

    def step(self):
        import spira_amd
        self.cache.reset()
        x = spira_amd.SparseTensor(coordinates=self.coords, features=self.feats, double=True)
        x.order()
        self.cache.add_all_kernel_maps(x._coordinates, self.ks, self.ss, self.ts, (1, 1, 1), self.dataflows)
        return self.model(x)

    def time(self, steps, warmup):
        torch = self.torch
        with torch.no_grad():
            for _ in range(warmup):
                self.step()
            torch.cuda.synchronize()
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0 = time.perf_counter()
            s.record()
            for _ in range(steps):
                out = self.step()
            e.record()
            torch.cuda.synchronize()
            wall = (time.perf_counter() - t0) * 1e3 / steps
        return s.elapsed_time(e) / steps, wall, [o._features for o in out]


def layer_work(m, S, T, P, K):
    """Algorithmic bytes and flops of one layer launch: fp16 features read
    and written once, fp16 weights, the int32 map read once; 2 P C_in C_out
    flops (P valid pairs)."""
    cin, cout = m.in_channels, m.out_channels
    nbytes = 2.0 * (S * cin + T * cout) + 2.0 * K * cin * cout + (4.0 * K * T if K > 1 else 0.0)
    return nbytes, 2.0 * P * cin * cout


def per_layer_profile(torch, e2e: E2E, reps: int = 5):
    """Every convolution's in-network time: HIP events at the layer's
    boundaries inside full steps (mean over `reps` steps), with its shape,
    valid pairs and algorithmic work."""
    import spira_amd
    convs = [(n, m) for n, m in e2e.model.named_modules() if isinstance(m, spira_amd.nn.SparseConv)]
    rec = defaultdict(list)
    meta = {}
    timing = False

    def pre(name, mod, inputs):
        if timing:
            ev = torch.cuda.Event(enable_timing=True)
            ev.record()
            rec[name].append([ev, None])

    def post(name, mod, inputs, output):
        if timing:
            ev = torch.cuda.Event(enable_timing=True)
            ev.record()
            rec[name][-1][1] = ev
            return
        x = inputs[0]
        S, T = x._features.shape[0], output._features.shape[0]
        K = int(np.prod(mod.kernel_size))
        if mod.is_trivial:
            P = T
        else:
            key = ((tuple(output._stride), tuple(x._stride)) if mod.transposed
                   else (tuple(x._stride), tuple(output._stride))) + (tuple(mod.kernel_size),)
            entry = mod._kernel_map_cache._kernel_maps_cache[key]
            omap, Tf = entry[3], entry[2]  # the forward layer's map and targets
            os_layout = entry[0] or mod._tunable_config["map_dataflow"] == 0
            P = int((omap[:Tf] >= 0).sum().item()) if os_layout else int((omap[:, :Tf] >= 0).sum().item())
        meta[name] = {"S": S, "T": T, "P": P, "K": K, "stride": tuple(output._stride),
                      "cin": mod.in_channels, "cout": mod.out_channels,
                      "dataflow": mod._tunable_config["map_dataflow"], "transposed": mod.transposed,
                      "tuning": mod._tunable_config.get("os_tuning")}

    handles = []
    for n, m in convs:
        handles.append(m.register_forward_pre_hook(lambda mod, inp, n=n: pre(n, mod, inp)))
        handles.append(m.register_forward_hook(lambda mod, inp, out, n=n: post(n, mod, inp, out)))
    try:
        with torch.no_grad():
            timing = False
            e2e.step()  # shapes and valid pairs (reads back counts: not timed)
            timing = True
            for _ in range(reps):
                e2e.step()
        torch.cuda.synchronize()
    finally:
        for h in handles:
            h.remove()
    rows = []
    for n, m in convs:
        if n not in meta:
            continue
        ms = float(np.mean([a.elapsed_time(b) for a, b in rec[n]]))
        d = meta[n]
        nbytes, flops = layer_work(m, d["S"], d["T"], d["P"], d["K"])
        rows.append({"layer": n, **d, "ms": ms, "bytes": nbytes, "flops": flops})
    return rows


def family_name(key):
    return f"s{key[0]} {key[1]}->{key[2]} K{key[3]}"


def family_roofline(rows):
    """Group the layers by (stride, C_in, C_out, offsets); the family with the
    largest in-network time per step is the dominant one.  Its roofline: the
    binding bound of its summed algorithmic work (bytes at HBM peak vs flops
    at MFMA peak) against its summed time."""
    fam = defaultdict(lambda: {"ms": 0.0, "bytes": 0.0, "flops": 0.0, "launches": 0})
    for r in rows:
        key = (r["stride"][0], r["cin"], r["cout"], r["K"])
        f = fam[key]
        f["ms"] += r["ms"]
        f["bytes"] += r["bytes"]
        f["flops"] += r["flops"]
        f["launches"] += 1
    key, f = max(fam.items(), key=lambda kv: kv[1]["ms"])
    gbs = f["bytes"] / (f["ms"] * 1e-3) / 1e9
    tf = f["flops"] / (f["ms"] * 1e-3) / 1e12
    mfma_bound = f["flops"] / (MFMA_F16_PEAK_TFLOPS * 1e12) > f["bytes"] / (HBM_PEAK_GBS * 1e9)
    if mfma_bound:
        rl = {"bound": "mfma", "achieved": tf, "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
              "frac": tf / MFMA_F16_PEAK_TFLOPS}
    else:
        rl = {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS}
    rl.update({"traffic": MEASURED_TRAFFIC.get(family_name(key)),
               "kernel": f"os_kernel family: stride {key[0]}, {key[1]} -> {key[2]} channels, {key[3]} offsets "
                         f"({f['launches']} launches per step, in-network)",
               "ms_per_step": f["ms"], "algorithmic_bytes_per_step": f["bytes"],
               "algorithmic_flops_per_step": f["flops"], "hbm_gbs": gbs, "mfma_tflops": tf,
               "mfma_frac": tf / MFMA_F16_PEAK_TFLOPS, "hbm_frac": gbs / HBM_PEAK_GBS})
    fams = sorted(({"family": family_name(k), "key": k, "ms": v["ms"], "launches": v["launches"],
                    "mfma_frac": v["flops"] / (v["ms"] * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS,
                    "hbm_frac": v["bytes"] / (v["ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS}
                   for k, v in fam.items()), key=lambda d: -d["ms"])
    return rl, fams, key


def write_layer_table(path, rows, step_ms):
    lines = ["| # | layer | stride | C_in -> C_out | K | T | P | dataflow | in-network us | "
             "TFLOP/s | MFMA frac | GB/s | HBM frac |",
             "|---|---|---|---|---|---|---|---|---|---|---|---|---|"]
    for i, r in enumerate(rows):
        tf = r["flops"] / (r["ms"] * 1e-3) / 1e12
        gb = r["bytes"] / (r["ms"] * 1e-3) / 1e9
        lines.append(f"| {i} | {r['layer']} | {r['stride'][0]} | {r['cin']} -> {r['cout']} | {r['K']} | {r['T']} | "
                     f"{r['P']} | {r['dataflow']}{' (T)' if r['transposed'] else ''} | {r['ms'] * 1e3:.1f} | "
                     f"{tf:.0f} | {tf / MFMA_F16_PEAK_TFLOPS:.3f} | {gb:.0f} | {gb / HBM_PEAK_GBS:.3f} |")
    conv_ms = sum(r["ms"] for r in rows)
    lines.append("")
    lines.append(f"Convolutions: {conv_ms:.3f} ms of a {step_ms:.3f} ms step (layer-boundary events, so each "
                 f"row includes the layer's host launch gaps).")
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")


# ---------------------------------------------------------------------------
# config 2: kernel-map search
# ---------------------------------------------------------------------------
def kmap_leg(torch, keys):
    """build_kmap(dataflow=0) per call as the reference times it (HIP events
    around the Python call, host overhead included) and the search kernel
    alone (back-to-back launches from C++), k = 3 / 5, stride 1 / 2."""
    from spira_amd.nn import functional as F
    from spira_amd.nn.functional import _native
    out = {}
    for s in (1, 2):
        tgt = keys if s == 1 else F.downsample(keys, (2, 2, 2))
        S, T = keys.shape[0], tgt.shape[0]
        for k in (3, 5):
            api_ms = event_time(torch, lambda: F.build_kmap(keys, tgt, k, 1, 0), reps=20, warmup=3)
            kern_ms = _native._C.time_kmap_search(keys, tgt, (k, k, k), (1, 1, 1), 50)
            nbytes = 8 * S + 8 * T + 4 * k ** 3 * T
            # valid (target, offset) pairs per target: the scene's neighbour density
            P = int((F.build_kmap(keys, tgt, k, 1, 0)[2][:T] >= 0).sum().item())
            out[f"k{k}s{s}"] = {"api_us": api_ms * 1e3, "kernel_us": kern_ms * 1e3, "S": S, "T": T,
                                "P_over_T": round(P / max(T, 1), 3),
                                "algorithmic_bytes": nbytes, "gbs": nbytes / (kern_ms * 1e-3) / 1e9,
                                "frac": nbytes / (kern_ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
    return out


# ---------------------------------------------------------------------------
# config 3: one layer, every dataflow
# ---------------------------------------------------------------------------
def layer_leg(torch, keys, channels=(16, 32, 64, 128, 256), reps=10):
    """Per channel count C (C_in = C_out): each dataflow's layer call timed
    with HIP events around it (maps built beforehand, like the reference's
    layerwise experiment), the output-stationary kernel alone, and the
    selector's pick (the fastest dataflow)."""
    from spira_amd.nn import functional as F
    from spira_amd.nn.functional import _native
    dev = torch.device("cuda:0")
    S = T = keys.shape[0]
    maps = {d: F.build_kmap(keys, keys, 3, 1, d) for d in range(9)}
    P = int((maps[0][2][:T] >= 0).sum().item())
    out = {}
    for C in channels:
        g = torch.Generator().manual_seed(C)
        X = torch.randn(S, C, generator=g).half().to(dev)
        W = (torch.randn(27, C, C, generator=g) / np.sqrt(27 * C)).half().to(dev)
        calls = {
            "os": lambda: F.sparse_convolution_forward_os(S, T, maps[0][2], X, W),
            "ws_fused": lambda: F.sparse_convolution_forward_ws_merged(S, T, X, W, maps[1][5], maps[1][6],
                                                                       maps[1][3], maps[1][7], maps[1][8]),
            "ws_gather_gemm_scatter": lambda: F.sparse_convolution_forward_ws(S, T, X, W, maps[2][3], maps[2][4],
                                                                              maps[2][5], 16, 16, None, -1),
        }
        for d in (3, 5, 7):
            m = maps[d]
            calls[f"hybrid{d}"] = (lambda m=m, d=d: F.sparse_convolution_forward_hs_merged(
                S, T, X, W, m[5], m[6], m[3], None if d == 3 else m[2], m[7], m[8]))
        for d in (4, 6, 8):
            m = maps[d]
            calls[f"hybrid{d}"] = (lambda m=m, d=d: F.sparse_convolution_forward_hs(
                S, T, X, W, m[3], m[4], m[5], None if d == 4 else m[2], 16, 16))
        flops = 2.0 * P * C * C
        res = {}
        for name, fn in calls.items():
            ms = event_time(torch, fn, reps=reps)
            res[name] = {"ms": ms, "mfma_frac": flops / (ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS}
        kern = _native._C.time_conv_os(S, T, maps[0][2], X, W, 20)
        pick = min(res, key=lambda k: res[k]["ms"])
        nbytes = 2.0 * (S * C + T * C) + 2.0 * 27 * C * C + 4.0 * 27 * T
        out[str(C)] = {"dataflows": res, "selector_pick": pick, "selector_ms": res[pick]["ms"],
                       "os_kernel_ms": kern, "os_kernel_mfma_frac": flops / (kern * 1e-3) / 1e12 /
                       MFMA_F16_PEAK_TFLOPS, "os_kernel_hbm_frac": nbytes / (kern * 1e-3) / 1e9 / HBM_PEAK_GBS}
    return {"pairs": P, "voxels": S, "P_over_T": round(P / max(T, 1), 3), "per_C": out}


def kmap_floor_leg(torch, km):
    """The write-only floor of the map search: the library's -1 fill
    (spira_hip_fill_i32) over an int32 array of each config-2 map's size,
    timed like the search kernel (back-to-back launches between HIP events).
    A search must write its whole map, so this bounds its HBM fraction."""
    import ctypes
    lib = ctypes.CDLL(os.path.join(ROOT, "spira_amd", "libspira_hip.so"))
    lib.spira_hip_fill_i32.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p]
    dev = torch.device("cuda:0")
    out = {}
    for name, e in km.items():
        n = (e["algorithmic_bytes"] - 8 * e["S"] - 8 * e["T"]) // 4  # the map's int32 words (K T)
        x = torch.empty(n, dtype=torch.int32, device=dev)
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        ms = event_time(torch, lambda: lib.spira_hip_fill_i32(x.data_ptr(), n, -1, s), reps=50, warmup=5)
        out[name] = {"map_bytes": 4 * n, "fill_us": ms * 1e3,
                     "search_frac_bound": e["algorithmic_bytes"] / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
    return out


def config1_leg(torch, reps=20):
    """Config 1: one fp32 layer (20k voxels on spheres and planes in a 128^3
    grid, k = 3, C_in = C_out = 32), the output-stationary fp32 MFMA kernel
    timed through the API call and alone; also C = 64, 128 on the same map."""
    from spira_amd import scenes
    from spira_amd.nn import functional as F
    from spira_amd.nn.functional import _native
    dev = torch.device("cuda:0")
    coords = scenes.spheres_planes()
    keys, _ = F.flat_sort(torch.from_numpy(coords).to(dev), True)
    S = T = keys.shape[0]
    m = F.build_kmap(keys, keys, 3, 1, 0)[2]
    P = int((m[:T] >= 0).sum().item())
    out = {"voxels": S, "P_over_T": round(P / T, 3), "per_C": {}}
    for C in (32, 64, 128):
        g = torch.Generator().manual_seed(C)
        X = torch.randn(S, C, generator=g).to(dev)
        W = (torch.randn(27, C, C, generator=g) / np.sqrt(27 * C)).to(dev)
        api = event_time(torch, lambda: F.sparse_convolution_forward_os(S, T, m, X, W), reps=reps)
        kern = _native._C.time_conv_os(S, T, m, X, W, reps)
        flops = 2.0 * P * C * C
        dense = 2.0 * T * 27 * C * C
        out["per_C"][str(C)] = {"api_ms": api, "kernel_ms": kern,
                                "fp32_mfma_frac": flops / (kern * 1e-3) / 1e12 / MFMA_F32_PEAK_TFLOPS,
                                "dense_fp32_mfma_frac": dense / (kern * 1e-3) / 1e12 / MFMA_F32_PEAK_TFLOPS}
    return out


def family_leg(torch, indoor_np, rows, fams):
    """Every submanifold family's layer shape alone (random features and
    weights on the config-4 map of its stride, the in-network layer's tuned
    launch and row order), in a fixed order (by stride, then channels): 1 warm
    launch and 20 back-to-back launches each, the runs of identical dispatches
    the rocprofv3 counter passes read."""
    from spira_amd.nn import functional as F
    from spira_amd.nn.functional import _native
    dev = torch.device("cuda:0")
    out = {}
    keys, _ = F.flat_sort(torch.from_numpy(indoor_np).to(dev), True)
    for key in sorted(f["key"] for f in fams):
        stride, cin, cout, K = key
        layer = next(r for r in rows if (r["stride"][0], r["cin"], r["cout"], r["K"]) == key)
        if K != 27 or layer["transposed"] or layer["S"] != layer["T"]:
            continue
        ks = keys if stride == 1 else F.downsample(keys, (stride,) * 3)
        m = F.build_kmap(ks, ks, 3, stride, 0)
        T = int(ks.shape[0])
        X = torch.randn(T, cin, device=dev).half()
        W = (torch.randn(K, cin, cout, device=dev) / np.sqrt(K * cin)).half()
        tuning = layer["tuning"]
        ms = _native._C.time_conv_os(T, T, m[2], X, W, 20, tuning=tuning)
        plan = _native._C.conv_os_plan(T, K, cin, 0, cout, True, tuning)
        out[family_name(key)] = {"kernel_ms": ms, "T": T, "grid": [plan[4], plan[5]],
                                 "tuning": list(tuning) if tuning else None,
                                 "traffic": MEASURED_TRAFFIC.get(family_name(key))}
    return out


def c5family_leg(torch, blobs_np):
    """Config 5's 125-offset submanifold layer shapes, one per level (16, 32,
    64, 128 channels at strides 1, 2, 4, 8), each alone on the config-5 map of
    its stride with random features and weights at the library's default
    launch: 1 warm launch and 20 back-to-back launches each, in that order
    (the runs of identical dispatches the rocprofv3 counter passes read)."""
    from spira_amd.nn import functional as F
    from spira_amd.nn.functional import _native
    dev = torch.device("cuda:0")
    out = {}
    keys, _ = F.flat_sort(torch.from_numpy(blobs_np).to(dev), True)
    for stride, c in ((1, 16), (2, 32), (4, 64), (8, 128)):
        ks = keys if stride == 1 else F.downsample(keys, (stride,) * 3)
        m = F.build_kmap(ks, ks, 5, stride, 0)[2]
        T = int(ks.shape[0])
        P = int((m >= 0).sum())
        X = torch.randn(T, c, device=dev).half()
        W = (torch.randn(125, c, c, device=dev) / np.sqrt(125 * c)).half()
        ms = _native._C.time_conv_os(T, T, m, X, W, 20)
        plan = _native._C.conv_os_plan(T, 125, c, 0, c, True, None)
        flops = 2.0 * P * c * c
        out[f"s{stride} {c}->{c} K125"] = {"kernel_ms": ms, "T": T, "P_over_T": round(P / T, 2),
                                           "plan": list(plan), "mfma_frac": flops / (ms * 1e-3) / 1e12 /
                                           MFMA_F16_PEAK_TFLOPS}
    return out


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


def rel_err(got, ref):
    rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2))) or 1.0
    return float(np.max(np.abs(got.astype(np.float64) - ref))) / rms


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: every GPU box here has one MI355X; "
                                   "use --gpus 1"}))
        sys.exit(2)
    import torch
    from spira_amd import scenes
    from spira_amd.nn import functional as F

    if args.concurrent_maps:
        from spira_amd.nn.functional import _native
        _native._C.set_concurrent_maps(True)
    legs = set(args.only.split(",")) if args.only else {"e2e", "kmap", "layer", "config5", "config1"}
    with open(os.path.join(ROOT, "BASELINE.json")) as f:
        baseline = json.load(f)
    dev = torch.device("cuda:0")

    indoor = scenes.indoor()
    res = {"metric": baseline["metric"], "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
           "data": "synthetic (seeded scenes, random-init weights)"}
    cfg = {"workload": "config4: SparseResUNet42 fp16, 200k-voxel indoor scene, end-to-end "
                       "(order + network-wide kernel maps + forward; selector run before timing)",
           "voxels": int(indoor.shape[0]), "key_bits": 64, "concurrent_maps": bool(args.concurrent_maps)}
    cpu = {}
    e2e = None
    if "e2e" in legs or "family" in legs:
        e2e = E2E(torch, args, indoor, "UNet")
        if not args.no_tune:
            res["untuned_ms_per_step"], _, _ = e2e.time(min(args.steps, 10), min(args.warmup, 5))
            e2e.tune()
        ms, wall, gpu_out = e2e.time(args.steps, args.warmup)
        res["value"] = ms
        res["ms_per_step"] = ms
        res["wall_ms_per_step"] = wall
        cfg["map_dataflows"] = e2e.dataflows
        if e2e.chosen:
            cfg["row_orders"] = e2e.chosen["row_orders"]
        rows = per_layer_profile(torch, e2e)
        rl, fams, fkey = family_roofline(rows)
        res["roofline"] = rl
        res["families"] = fams[:6]
        cfg["levels"] = {f"s{r['stride'][0]}": {"T": r["T"], "P_over_T": round(r["P"] / r["T"], 2)}
                         for r in rows if r["K"] == 27 and not r["transposed"]}
        if args.layer_table:
            write_layer_table(args.layer_table, rows, ms)
        if "family" in legs:
            res["family_kernels"] = family_leg(torch, indoor, rows, fams)
        if not args.no_cpu:
            # the same network, weights and input features through the oracle
            # (fp32) on the host cores, timed; outputs checked against the GPU's
            from oracle import oracle as orc
            from oracle.network import network_forward
            feats = e2e.feats.float().cpu().numpy()
            t0 = time.perf_counter()
            ref = network_forward(e2e.model, indoor, feats)
            cpu_ms = (time.perf_counter() - t0) * 1e3
            errs = [rel_err(g.float().cpu().numpy(), rf) for g, (rf, _) in zip(gpu_out, ref)]
            res["cpu_baseline"] = {"value": cpu_ms, "unit": "ms", "cores": orc.threads(), "kind": "port",
                                   "sample": "one full config-4 step (sort, downsample, all maps, all 42 layers, "
                                             "fp32) by the OpenMP oracle, on the GPU run's weights and inputs",
                                   "max_err_vs_gpu_x_rms": max(errs), "levels_compared": len(errs)}
    if "config5" in legs:
        # config 5: the large-kernel (k = 5) SparseResNetLarge on the ~300k-voxel
        # scene of merged LiDAR rings and Gaussian blobs, timed like config 4
        blobs = scenes.lidar_blobs()
        c5 = E2E(torch, args, blobs, "ResNetLarge")
        if not args.no_tune:
            res["config5_untuned_ms"], _, _ = c5.time(5, 3)
            c5.tune()
        res["config5_ms"], _, _ = c5.time(10, 5)
        cfg["config5_voxels"] = int(blobs.shape[0])
        del c5
    if "c5family" in legs:
        res["config5_families"] = c5family_leg(torch, scenes.lidar_blobs())
    if "kmap" in legs or "layer" in legs:
        lidar = scenes.lidar()
        lkeys, _ = F.flat_sort(torch.from_numpy(lidar).to(dev), True)
        cfg["kmap_voxels"] = int(lkeys.shape[0])
    if "kmap" in legs:
        km = kmap_leg(torch, lkeys)
        res["kmap"] = km
        res["kmap_write_floor"] = kmap_floor_leg(torch, km)
        res["kmap_build_us"] = km["k3s1"]["api_us"]
        res["kmap_kernel_us"] = km["k3s1"]["kernel_us"]
        res["kmap_roofline"] = {"bound": "hbm", "achieved": km["k3s1"]["gbs"], "peak": HBM_PEAK_GBS,
                                "unit": "GB/s", "frac": km["k3s1"]["frac"], "traffic": KMAP_TRAFFIC,
                                "kernel": "kmap_search_kernel<u64,3,3,0> (config 2, k=3, stride 1, OS layout)",
                                "algorithmic_bytes": km["k3s1"]["algorithmic_bytes"]}
        if not args.no_cpu:
            from oracle import oracle as orc
            kn = lkeys.cpu().numpy()
            t0 = time.perf_counter()
            ref = orc.search(kn, kn, (3, 3, 3), (1, 1, 1), orc.OS)
            cpu_ms = (time.perf_counter() - t0) * 1e3
            got = F.build_kmap(lkeys, lkeys, 3, 1, 0)[2].cpu().numpy()
            cpu["kmap_k3s1"] = {"value": cpu_ms * 1e3, "unit": "us", "cores": orc.threads(), "kind": "port",
                                "sample": "the config-2 k=3 stride-1 map (output-stationary layout)",
                                "bit_exact_vs_gpu": bool(np.array_equal(got, ref))}
    if "layer" in legs:
        ly = layer_leg(torch, lkeys)
        res["layers"] = ly
        res["layer_ms"] = ly["per_C"]["64"]["selector_ms"]
        if not args.no_cpu:
            from oracle import oracle as orc
            C = 64
            kn = lkeys.cpu().numpy()
            omap = orc.search(kn, kn, (3, 3, 3), (1, 1, 1), orc.OS)
            g = torch.Generator().manual_seed(C)
            X = torch.randn(kn.shape[0], C, generator=g).half()
            W = (torch.randn(27, C, C, generator=g) / np.sqrt(27 * C)).half()
            t0 = time.perf_counter()
            ref = orc.conv_os_f32(omap, kn.shape[0], X.float().numpy(), W.float().numpy())
            cpu_ms = (time.perf_counter() - t0) * 1e3
            got = F.sparse_convolution_forward_os(kn.shape[0], kn.shape[0], torch.from_numpy(omap).to(dev),
                                                  X.to(dev), W.to(dev)).float().cpu().numpy()
            cpu["layer_c64"] = {"value": cpu_ms, "unit": "ms", "cores": orc.threads(), "kind": "port",
                                "sample": "one config-3 C=64 layer (fp32 sums)", "max_err_vs_gpu_x_rms":
                                rel_err(got, ref)}
    if "config1" in legs:
        c1 = config1_leg(torch)
        res["config1_fp32"] = c1
        res["config1_fp32_ms"] = c1["per_C"]["32"]["api_ms"]
    if cpu:
        res["cpu_baselines"] = cpu
    if "calib" in legs:
        res["calib"] = calib_leg(torch)
    res["config"] = cfg
    print(json.dumps(res))


if __name__ == "__main__":
    main()
