"""FFI fwd + bwd + SR-SGD step throughput on one MI355X (BASELINE.json metric).

One step = forward logits (incl. the X -> X^T copy), backward to features
(deterministic, fused SR to bf16 with seed 123), and backward to weights and
bias (fp32, kept on chip) fused with the SR-SGD update of weights and bias
(lr 0.05, wd 1e-4, momentum 0, seed 42 + step; bit-identical to separate
gradient and SGD kernels, whose step time is reported as "unfused").  Inputs are synthetic and
resident in HBM before timing; the grad of the logits dY = bf16(sigmoid(z) - Y)
is computed once from the initial logits (Y binary,
~5 positives per row, Zipf(1.1) over labels).  "fused_loss" times the step a
training loop runs instead: the forward computes dY = sigma(z) - Y and the BCE
loss from the COO labels in its epilogue (no logits written), then the same
backward and update.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 1]
                       [--no-cpu-baseline] [--phases]
Prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "FFI fwd+bwd+SR-step samples/sec at O=131K/670K/3M; %HBM & %MFMA roofline"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0

CONFIGS = {
    0: dict(B=64, D=768, O=4096, G=32, F=32, pos=5),
    1: dict(B=512, D=768, O=131073, G=64, F=128, pos=5),
    2: dict(B=512, D=768, O=670091, G=64, F=64, pos=5),
    3: dict(B=256, D=4096, O=500000, G=32, F=256, pos=5),
    4: dict(B=1024, D=768, O=3000000, G=128, F=128, pos=10),
}


def phase_bytes(B, D, O, G, F):
    """Algorithmic HBM bytes per phase (bf16 tensors, momentum 0): every tensor
    read or written once.  bwd_weights_sgd keeps the fp32 gradients on chip:
    dY, X, idx read, W and bias read and written.  The unfused phases
    (bwd_weights writing fp32 dW/dbias, sgd reading them) are listed too."""
    Gc = (O + G - 1) // G
    return {
        "fwd": 2 * B * O + 2 * O * F + 4 * Gc * F + 2 * B * D + 2 * O,
        "bwd_features": 2 * B * O + 2 * O * F + 4 * Gc * F + 2 * B * D,
        "bwd_weights_sgd": 2 * B * O + 2 * B * D + 4 * Gc * F + (2 + 2) * O * F + (2 + 2) * O,
        "bwd_weights": 2 * B * O + 2 * B * D + 4 * Gc * F + 4 * O * F + 4 * O,
        "sgd": (2 + 4 + 2) * O * F + (2 + 4 + 2) * O,
    }


TRAFFIC_FILE = "profiles/traffic_config%d.txt"
COPY_BYTES = 256 * 1024 * 1024


def measured_traffic(config, phase):
    """HBM bytes per launch of ``phase`` from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (lines ``TRAFFIC <phase> <bytes>``), or None if absent."""
    path = os.path.join(ROOT, TRAFFIC_FILE % config)
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            parts = line.split()
            if len(parts) == 3 and parts[0] == "TRAFFIC" and parts[1] == phase:
                return float(parts[2])
    return None


def make_inputs(cfg, dev):
    import numpy as np
    import torch

    B, D, O, G, F = cfg["B"], cfg["D"], cfg["O"], cfg["G"], cfg["F"]
    Gc = (O + G - 1) // G
    x = torch.randn(B, D, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
    bound = 1.0 / math.sqrt(F)
    W = ((torch.rand(O, F, generator=torch.Generator().manual_seed(1)) * 2 - 1) * bound).to(torch.bfloat16)
    rng = np.random.default_rng(2)
    idx = np.argsort(rng.random((Gc, D), dtype=np.float32), axis=1)[:, :F].astype(np.int32)
    rng_y = np.random.default_rng(3)
    n_pos = B * cfg["pos"]
    lab = rng_y.zipf(1.1, size=4 * n_pos)
    lab = lab[lab <= O][:n_pos] - 1
    rows = np.repeat(np.arange(B), cfg["pos"])[: len(lab)]
    Y = torch.zeros(B, O, dtype=torch.float32)
    Y[torch.from_numpy(rows), torch.from_numpy(lab)] = 1.0
    return (x.to(dev), W.to(dev), torch.zeros(O, dtype=torch.bfloat16, device=dev),
            torch.from_numpy(idx).to(dev), Y.to(dev))


def make_labels(cfg, dev):
    """The positives of make_inputs' Y as COO int32 [nnz, 2] (row, label) pairs
    (the application's label format, src/data.py:26-46)."""
    import numpy as np
    import torch

    B, O = cfg["B"], cfg["O"]
    rng_y = np.random.default_rng(3)
    n_pos = B * cfg["pos"]
    lab = rng_y.zipf(1.1, size=4 * n_pos)
    lab = lab[lab <= O][:n_pos] - 1
    rows = np.repeat(np.arange(B), cfg["pos"])[: len(lab)]
    coo = np.unique(np.stack([rows, lab], 1).astype(np.int32), axis=0)  # Y is binary
    return torch.from_numpy(coo).to(dev)


def cpu_baseline(cfg, budget_s=20.0):
    """Times the CPU oracle (PyTorch-CPU gather+bmm fwd/bwd + C SR-SGD) on a
    slice of the label groups, scaled to the full label count."""
    import numpy as np
    import torch

    import oracle

    ncores = min(len(os.sched_getaffinity(0)), 16)
    torch.set_num_threads(ncores)
    oracle.set_num_threads(ncores)
    B, D, O, G, F = cfg["B"], cfg["D"], cfg["O"], cfg["G"], cfg["F"]
    Gc = (O + G - 1) // G
    frac = 1
    while Gc // frac > 256 and frac < 64:
        frac *= 2
    Gs = max(1, Gc // frac)
    Os = Gs * G
    g = torch.Generator().manual_seed(0)
    x = torch.randn(B, D, generator=g).to(torch.bfloat16)
    W = ((torch.rand(Os, F, generator=g) * 2 - 1) / math.sqrt(F)).to(torch.bfloat16)
    bias = torch.zeros(Os, dtype=torch.bfloat16)
    idx = torch.randint(0, D, (Gs, F), generator=g, dtype=torch.int32)
    dY = (torch.randn(B, Os, generator=g) * 0.1).to(torch.bfloat16)

    def one_step(seed):
        xT = x.t().contiguous()
        oracle.ffi_forward(idx, xT, W, bias, G).to(torch.bfloat16)
        dxt = oracle.ffi_backward_features(idx, W, dY, G, D)
        oracle.sr_round_bf16(dxt.t().contiguous().numpy(), 123)
        dW = oracle.ffi_backward_weights(idx, xT, dY, G)
        db = oracle.bias_grad(dY)
        wb = W.view(torch.int16).numpy().view(np.uint16)
        oracle.sgd_sr_step(wb, dW.numpy(), None, 0.05, 1e-4, 0.0, False, True, seed)
        oracle.sgd_sr_step(bias.view(torch.int16).numpy().view(np.uint16), db.numpy(), None,
                           0.05, 1e-4, 0.0, False, True, seed)

    one_step(0)  # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 and (time.perf_counter() - t_start) < budget_s:
        t0 = time.perf_counter()
        one_step(len(times) + 1)
        times.append(time.perf_counter() - t0)
    t_med = sorted(times)[len(times) // 2]
    t_full = t_med * (O / Os)
    return {"value": B / t_full, "unit": "samples/s", "cores": ncores, "kind": "port",
            "sample": (f"oracle (torch-CPU gather+bmm fwd/bwd + C/OpenMP SR-SGD) on {Gs} of {Gc} "
                       f"label groups (O_s={Os}), median of {len(times)} steps after 1 warm-up, "
                       f"step time scaled by O/O_s={O / Os:.1f}"),
            "step_ms_full_scaled": t_full * 1e3}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=1, choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--phases", action="store_true",
                    help="also print per-phase event timings to stderr")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="after the timed steps, copy a 256 MiB fp32 buffer 3 times (a kernel "
                         "of known traffic for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU: the FFI path shards by label "
                          "groups with one all-reduce of dX per step (see DESIGN.md); "
                          "multi-GPU runs are not part of this build", "n_gpus": args.gpus}))
        sys.exit(2)

    import torch

    from haste_amd.step import FFITrainStep

    dev = torch.device("cuda:0")
    cfg = CONFIGS[args.config]
    B, D, O, G, F = cfg["B"], cfg["D"], cfg["O"], cfg["G"], cfg["F"]
    x, W, bias, idx, Y = make_inputs(cfg, dev)
    st = FFITrainStep(W, bias, idx, B, D, G, lr=0.05, weight_decay=1e-4, seed=42)
    logits = st.forward(x)
    ldy = st.ldo
    dY_buf = torch.zeros(B, ldy, dtype=torch.bfloat16, device=dev)
    dY_buf[:, :O] = (torch.sigmoid(logits.float()) - Y).to(torch.bfloat16)
    labels = make_labels(cfg, dev)  # the same positives as COO (row, label) pairs
    del Y
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream()
    names = ["fwd", "bwd_features", "bwd_weights_sgd"]
    fns = [lambda: st.forward(x), lambda: st.backward_features(dY_buf, ldy),
           lambda: st.backward_weights_sgd(dY_buf, ldy)]

    def timed(fn_list, steps, warmup):
        """(ms per step, per-phase ms, wall s).  The step time comes from K steps with
        nothing but the two bracketing events; the per-phase times from a second
        pass of K steps with an event between phases (recording events between
        kernels adds gaps, so those phases sum to more than the step time)."""
        for _ in range(warmup):
            for fn in fn_list:
                fn()
        torch.cuda.synchronize()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        w0 = time.perf_counter()
        for _ in range(steps):
            for fn in fn_list:
                fn()
        t1.record(stream)
        torch.cuda.synchronize()
        wall_s = time.perf_counter() - w0
        evs = [[torch.cuda.Event(enable_timing=True) for _ in range(len(fn_list) + 1)]
               for _ in range(steps)]
        for k in range(steps):
            evs[k][0].record(stream)
            for i, fn in enumerate(fn_list):
                fn()
                evs[k][i + 1].record(stream)
        torch.cuda.synchronize()
        per = [sum(e[i].elapsed_time(e[i + 1]) for e in evs) / steps for i in range(len(fn_list))]
        return t0.elapsed_time(t1) / steps, per, wall_s

    ms_per_step, per, wall = timed(fns, args.steps, args.warmup)
    phase_ms = dict(zip(names, per))
    # the same step with separate gradient and SGD kernels (identical results)
    un_names = ["fwd", "bwd_features", "bwd_weights", "sgd"]
    un_ms, un_per, _ = timed([lambda: st.forward(x), lambda: st.backward_features(dY_buf, ldy),
                              lambda: st.backward_weights(dY_buf, ldy), st.sgd],
                             max(5, args.steps // 2), 2)

    # the step with the loss fused into the forward (dY from the labels; the logits
    # are not written): what a training loop runs per batch
    fl_names = ["fwd_bce", "bwd_features", "bwd_weights_sgd"]
    fl_ms, fl_per, _ = timed([lambda: st.forward_bce(x, labels),
                              lambda: st.backward_features(st.dY_buf, ldy),
                              lambda: st.backward_weights_sgd(st.dY_buf, ldy)],
                             max(5, args.steps // 2), 2)

    pb = phase_bytes(B, D, O, G, F)
    phase_gbs = {n: pb[n] / (phase_ms[n] * 1e-3) / 1e9 for n in names}
    dom = max(names, key=lambda n: phase_ms[n])
    step_bytes = sum(pb[n] for n in names)
    flops = 3 * 2 * B * O * F
    result = {
        "metric": METRIC,
        "value": B / (ms_per_step * 1e-3),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"BASELINE config {args.config}: grouped FFI fwd + bwd_features + "
                               f"bwd_weights + SR-SGD step", "B": B, "D": D, "O": O, "G": G,
                   "fan_in": F, "grad_dtype": "fp32"},
        "roofline": {"bound": "hbm", "achieved": phase_gbs[dom], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": phase_gbs[dom] / HBM_PEAK_GBS, "traffic": None,
                     "kernel_phase": dom},
        "step_roofline": {"bytes": step_bytes, "hbm_frac": step_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS,
                          "mfma_frac": flops / (ms_per_step * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS},
        "phases_us": {n: round(phase_ms[n] * 1e3, 2) for n in names},
        "phases_hbm_frac": {n: round(phase_gbs[n] / HBM_PEAK_GBS, 4) for n in names},
        "unfused": {"ms_per_step": un_ms, "samples_per_s": B / (un_ms * 1e-3),
                    "phases_us": {n: round(v * 1e3, 2) for n, v in zip(un_names, un_per)}},
        "fused_loss": {"ms_per_step": fl_ms, "samples_per_s": B / (fl_ms * 1e-3),
                       "phases_us": {n: round(v * 1e3, 2) for n, v in zip(fl_names, fl_per)},
                       "workload": "forward + sparse BCE gradient from COO labels (loss summed "
                                   "on the device, logits not written) + bwd_features + "
                                   "bwd_weights + SR-SGD"},
        "wall_s": wall,
    }
    tr = measured_traffic(args.config, dom)
    if tr is not None:
        result["roofline"]["traffic"] = tr
        result["roofline"]["traffic_source"] = TRAFFIC_FILE % args.config
    if args.copy_calibration:
        src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(cfg)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
