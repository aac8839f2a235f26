"""FFI fwd + bwd + SR-SGD step throughput on one MI355X (BASELINE.json metric).

One step = forward logits (incl. the X -> X^T copy), backward to features
(deterministic, SR to bf16 with seed 123), and backward to weights and bias
(fp32, kept on chip) fused with the SR-SGD update of weights and bias (lr 0.05,
wd 1e-4, momentum 0, seed 42 + step; bit-identical to separate gradient and SGD
kernels, whose step time is reported as "unfused"); the launch of the update
also runs the final pass of backward to features (the sum of its per-slice
partials into dX).

Warm-up: W steps, continued until the GPU has run the step for WARM_MS
(the MI355X reaches its steady clock after about 25 ms of sustained load; the
step time then stays flat for seconds), then exactly K timed steps.  Inputs are
synthetic and resident in HBM before timing; the grad of the logits
dY = bf16(sigmoid(z) - Y) is computed once from the initial logits (BASELINE
configs: Y binary, ~5 positives per row (10 at config 4), Zipf(1.1) over
labels).  "hip_graph" is the same step captured once in a HIP graph and
replayed (the SR-SGD seed is read and advanced on the device).  "fused_loss"
times the step a training loop runs instead: the
forward computes dY = sigma(z) - Y and the BCE loss from the COO labels in its
epilogue (no logits written), then the same backward and update.

The headline (``value``) is config 1 (--config).  The same line carries:
  * "configs": the step at BASELINE configs 2, 3 and 4 (O = 670K / 500K / 3M),
    each with per-phase times and %HBM; at configs 2 and 4 also their rewire
    (prune 15 % per group by mean |W|, regrow unused indices, zero init; every
    1000 steps in the reference's runs) timed alone and with the index re-plan
    it costs the next step, raw and amortised over 1000 steps;
  * "dropin_api": the reference's own API path at config 1 (GroupFixedFanIn
    forward, autograd backward with dX, SRSgd.step), bf16 and fp32 gradients;
  * "sr_floor": the phases that round stochastically (the fused update, and the
    unfused SGD) against both of their floors: HBM (algorithmic bytes at the
    peak) and the Philox arithmetic of one tl.randint word per element, timed
    live with haste_sr_words_fold (the words alone);
  * "cpu_baseline": the CPU oracle's step (PyTorch-CPU gather + bmm, C/OpenMP
    SR-SGD) on all the host cores in this process's affinity.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 1]
                       [--extra-configs 2,3,4] [--no-dropin] [--no-cpu-baseline]
                       [--copy-calibration]
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
LR, WD, SEED = 0.05, 1e-4, 42
REWIRE_FRACTION, REWIRE_INTERVAL = 0.15, 1000
REWIRE_CONFIGS = (2, 4)  # the BASELINE configs that include a rewire step

CONFIGS = {
    0: dict(B=64, D=768, O=4096, G=32, F=32, pos=5),
    1: dict(B=512, D=768, O=131073, G=64, F=128, pos=5),
    2: dict(B=512, D=768, O=670091, G=64, F=64, pos=5),
    3: dict(B=256, D=4096, O=500000, G=32, F=256, pos=5),
    4: dict(B=1024, D=768, O=3000000, G=128, F=128, pos=10),
}


def phase_bytes(B, D, O, G, F):
    """Algorithmic HBM bytes per phase (bf16 tensors, momentum 0): every tensor
    read or written once.  The step's bwd_features reads dY, W and idx and leaves
    dX (its per-slice partials) to bwd_weights_sgd, whose launch writes it; that
    phase keeps the fp32 gradients on chip: dY, X, idx read, W and bias read and
    written, dX written.  The unfused phases (bwd_weights writing fp32
    dW/dbias, sgd reading them) are listed too."""
    Gc = (O + G - 1) // G
    return {
        "fwd": 2 * B * O + 2 * O * F + 4 * Gc * F + 2 * B * D + 2 * O,
        "bwd_features": 2 * B * O + 2 * O * F + 4 * Gc * F,
        "bwd_weights_sgd": (2 * B * O + 2 * B * D + 4 * Gc * F + (2 + 2) * O * F + (2 + 2) * O
                            + 2 * B * D),
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


def positives(cfg):
    """Y's positives as unique (row, label) pairs: ``pos`` per row, labels drawn
    Zipf(1.1) (numpy seed 3)."""
    import numpy as np

    B, O = cfg["B"], cfg["O"]
    rng_y = np.random.default_rng(3)
    n_pos = B * cfg["pos"]
    lab = rng_y.zipf(1.1, size=4 * n_pos)
    lab = lab[lab <= O][:n_pos] - 1
    rows = np.repeat(np.arange(B), cfg["pos"])[: len(lab)]
    return np.unique(np.stack([rows, lab], 1).astype(np.int32), axis=0)


def make_inputs(cfg, dev):
    """x bf16 N(0,1) [B, D]; W bf16 U(+-1/sqrt(F)) [O, F]; bias 0; idx int32
    [Gc, F], F distinct features per group (numpy seed 2); generated on the
    device (torch seeds 0 and 1) so that the 3M-label config needs no host copy."""
    import numpy as np
    import torch

    B, D, O, G, F = cfg["B"], cfg["D"], cfg["O"], cfg["G"], cfg["F"]
    Gc = (O + G - 1) // G
    x = torch.randn(B, D, generator=torch.Generator(device=dev).manual_seed(0),
                    device=dev).to(torch.bfloat16)
    W = torch.rand(O, F, generator=torch.Generator(device=dev).manual_seed(1), device=dev)
    W = W.mul_(2).sub_(1).mul_(1.0 / math.sqrt(F)).to(torch.bfloat16)
    rng = np.random.default_rng(2)
    idx = np.empty((Gc, F), dtype=np.int32)
    for g0 in range(0, Gc, 4096):  # bounded host memory at config 4
        g1 = min(Gc, g0 + 4096)
        idx[g0:g1] = np.argsort(rng.random((g1 - g0, D), dtype=np.float32), axis=1)[:, :F]
    return x, W, torch.zeros(O, dtype=torch.bfloat16, device=dev), torch.from_numpy(idx).to(dev)


def make_dY(logits, pos, lddy, dev):
    """dY = bf16(sigmoid(z) - Y) in a [B, lddy] buffer (zero padding), rows in
    chunks so the fp32 temporaries stay small."""
    import torch

    B, O = logits.shape
    dY = torch.zeros(B, lddy, dtype=torch.bfloat16, device=dev)
    for r0 in range(0, B, 128):
        dY[r0:r0 + 128, :O] = torch.sigmoid(logits[r0:r0 + 128].float()).to(torch.bfloat16)
    p = torch.from_numpy(pos).to(dev).long()
    z = logits[p[:, 0], p[:, 1]].float()
    dY[p[:, 0], p[:, 1]] = (torch.sigmoid(z) - 1.0).to(torch.bfloat16)
    return dY


WARM_MS = 50.0


def warm_up(fn_list, warmup):
    """Run at least ``warmup`` steps, and more until WARM_MS of wall time (the host
    syncs every 10 steps past ``warmup``, so that is GPU time); returns the count."""
    import torch

    w0 = time.perf_counter()
    n = 0
    while n < warmup or (time.perf_counter() - w0) * 1e3 < WARM_MS:
        for fn in fn_list:
            fn()
        n += 1
        if n >= warmup and n % 10 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return n


def timed(fn_list, steps, warmup, stream):
    """(ms per step, per-phase ms, wall s).  The step time comes from K steps with
    nothing but the two bracketing events (on the stream every kernel runs on);
    the per-phase times from a second pass of K steps with an event between phases
    (recording events between kernels adds gaps, so those phases sum to more than
    the step time)."""
    import torch

    warm_up(fn_list, warmup)
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


NAMES = ["fwd", "bwd_features", "bwd_weights_sgd"]


def setup_step(cfg, dev):
    import torch

    from haste_amd.step import FFITrainStep

    x, W, bias, idx = make_inputs(cfg, dev)
    st = FFITrainStep(W, bias, idx, cfg["B"], cfg["D"], cfg["G"], lr=LR, weight_decay=WD,
                      seed=SEED)
    logits = st.forward(x)
    pos = positives(cfg)
    dY = make_dY(logits, pos, st.ldo, dev)
    torch.cuda.synchronize()
    return st, x, dY, pos


def step_fns(st, x, dY):
    return [lambda: st.forward(x), lambda: st.backward_features(dY, st.ldo, defer_dx=True),
            lambda: st.backward_weights_sgd(dY, st.ldo)]


def sr_word_rate(dev, n=1 << 26, reps=5):
    """tl.randint words per second of haste_sr_words_fold, the Philox4x32-10
    arithmetic of the SR and SR-SGD kernels alone (one word per weight, fixed
    by bit-exact parity with tl.randint), timed with events on the stream it
    runs on."""
    import torch

    from haste_amd import _C, _lib

    fold = torch.empty((n + 63) // 64, dtype=torch.int32, device=dev)
    st = _C.stream_of(fold)
    for _ in range(2):
        _lib.call("haste_sr_words_fold", fold.data_ptr(), n, SEED, st)
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        _lib.call("haste_sr_words_fold", fold.data_ptr(), n, SEED, st)
    e1.record(stream)
    torch.cuda.synchronize()
    return n * reps / (e0.elapsed_time(e1) * 1e-3)


def sr_words(B, D, O, F):
    """Random words per launch of the phases that round stochastically: the fused
    update draws one per weight and bias element and one per dX element (its
    trailing workgroups round dX); the unfused SGD one per weight and bias."""
    return {"bwd_weights_sgd": O * F + O + B * D, "sgd": O * F + O}


def sr_floor_report(cfg, phases_ms, word_rate):
    """For each SR phase: the HBM floor (its algorithmic bytes at the peak), the
    Philox floor (its words at the measured word rate), and the phase time as a
    fraction of the larger one."""
    B, D, O, F, G = cfg["B"], cfg["D"], cfg["O"], cfg["F"], cfg["G"]
    pb, words = phase_bytes(B, D, O, G, F), sr_words(B, D, O, F)
    out = {}
    for name, ms in phases_ms.items():
        if name not in words:
            continue
        hbm_us = pb[name] / (HBM_PEAK_GBS * 1e9) * 1e6
        valu_us = words[name] / word_rate * 1e6
        floor = max(hbm_us, valu_us)
        out[name] = {"words": words[name], "hbm_floor_us": round(hbm_us, 2),
                     "valu_floor_us": round(valu_us, 2),
                     "bound": "valu" if valu_us > hbm_us else "hbm",
                     "measured_us": round(ms * 1e3, 2), "frac_of_floor": round(floor / (ms * 1e3), 4)}
    return out


def phase_report(cfg, ms_per_step, per):
    B, D, O, G, F = cfg["B"], cfg["D"], cfg["O"], cfg["G"], cfg["F"]
    pb = phase_bytes(B, D, O, G, F)
    step_bytes = sum(pb[n] for n in NAMES)
    return {
        "ms_per_step": ms_per_step,
        "samples_per_s": B / (ms_per_step * 1e-3),
        "phases_us": {n: round(v * 1e3, 2) for n, v in zip(NAMES, per)},
        "phases_hbm_frac": {n: round(pb[n] / (v * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
                            for n, v in zip(NAMES, per)},
        "step_hbm_frac": step_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "step_mfma_frac": 3 * 2 * B * O * F / (ms_per_step * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
    }


def time_rewire(st, x, dY, cfg, stream, reps=5):
    """The reference's rewire at this config (rewire.py:143-239 semantics of the
    build: prune the int(F * 0.15) smallest mean-|W| slots per group, regrow
    unused indices, zero init), timed alone, and with the cost it adds to the
    next step (the bwd-features index plan and transposed weights are rebuilt
    once after idx changes)."""
    import torch

    from haste_amd import _C, _lib

    F, G, D, O = cfg["F"], cfg["G"], cfg["D"], cfg["O"]
    k = int(F * REWIRE_FRACTION)
    n_pruned = torch.zeros(1, dtype=torch.int32, device=st.W.device)

    def rewire(seed):
        _lib.call("haste_rewire", st.W.data_ptr(), st.code, st.idx.data_ptr(), None,
                  n_pruned.data_ptr(),
                  O, F, G, D, _lib.PRUNE_FRACTION, 0.0, k, _lib.REGROW_UNUSED, _lib.INIT_ZERO,
                  1.0 / math.sqrt(F), seed, _C.stream_of(st.W))
        torch.autograd.graph.increment_version(st.W)
        torch.autograd.graph.increment_version(st.idx)

    fns = step_fns(st, x, dY)
    alone, with_step, plain = [], [], []
    for r in range(reps):
        for f in fns:  # steady state: plan and W^T current
            f()
        e = [torch.cuda.Event(enable_timing=True) for _ in range(5)]
        e[0].record(stream)
        for f in fns:
            f()
        e[1].record(stream)
        rewire(1000 + r)
        e[2].record(stream)
        for f in fns:
            f()
        e[3].record(stream)
        torch.cuda.synchronize()
        plain.append(e[0].elapsed_time(e[1]))
        alone.append(e[1].elapsed_time(e[2]))
        with_step.append(e[2].elapsed_time(e[3]))
    med = lambda v: sorted(v)[len(v) // 2]
    t_rw, t_next, t_plain = med(alone), med(with_step), med(plain)
    total_us = (t_rw + max(0.0, t_next - t_plain)) * 1e3
    return {"rewire_us": round(t_rw * 1e3, 2),
            "next_step_extra_us": round(max(0.0, t_next - t_plain) * 1e3, 2),
            "total_us": round(total_us, 2),
            "amortised_us_per_step": round(total_us / REWIRE_INTERVAL, 3),
            "amortised_frac_of_step": round(total_us / REWIRE_INTERVAL / (t_plain * 1e3), 5),
            "pruned_per_call": int(n_pruned.item()) // reps,
            "interval": REWIRE_INTERVAL,
            "mode": f"fraction {REWIRE_FRACTION} per group (k={k}), regrow unused, init zero"}


def run_extra_config(c, steps, warmup, dev, word_rate):
    import torch

    cfg = CONFIGS[c]
    st, x, dY, _ = setup_step(cfg, dev)
    stream = torch.cuda.current_stream()
    ms, per, _ = timed(step_fns(st, x, dY), steps, warmup, stream)
    rep = {"B": cfg["B"], "D": cfg["D"], "O": cfg["O"], "G": cfg["G"], "fan_in": cfg["F"]}
    rep.update(phase_report(cfg, ms, per))
    rep["sr_floor"] = sr_floor_report(cfg, dict(zip(NAMES, per)), word_rate)
    if c in REWIRE_CONFIGS:
        rep["rewire"] = time_rewire(st, x, dY, cfg, stream)
    del st, x, dY
    torch.cuda.empty_cache()
    return rep


def time_dropin(cfg, steps, warmup, dev):
    """The reference's API path, one training step at a time: out =
    GroupFixedFanIn(x) (x requires grad), out.backward(dY) with dY the [B, O]
    gradient autograd hands over, SRSgd.step(), zero_grad()."""
    import torch

    from haste_amd.optim_sr import SRSgd
    from haste_amd.rewire import GroupFixedFanIn

    B, D, O, G, F = cfg["B"], cfg["D"], cfg["O"], cfg["G"], cfg["F"]
    x, W, bias, idx = make_inputs(cfg, dev)
    out = {}
    for mode in ("bf16_grads", "fp32_grads"):
        layer = GroupFixedFanIn(D, O, F, group_size=G, prune_mode="fraction",
                                rewire_fraction=REWIRE_FRACTION, dtype=torch.bfloat16,
                                device="cpu", fp32_grads=(mode == "fp32_grads"))
        layer = layer.to(dev)
        with torch.no_grad():
            layer.weights.copy_(W)
            layer.bias.copy_(bias)
            layer.group_locations.copy_(idx)
        opt = SRSgd(layer.parameters(), lr=LR, weight_decay=WD, momentum=0.0, seed=SEED)
        xr = x.detach().clone().requires_grad_(True)
        with torch.no_grad():
            logits = layer(xr)
        dY = make_dY(logits, positives(cfg), O, dev)[:, :O].contiguous()  # [B, O] as autograd's

        def one():
            opt.zero_grad()
            xr.grad = None
            layer(xr).backward(dY)
            opt.step()

        ms, _, _ = timed([one], steps, warmup, torch.cuda.current_stream())
        out[mode] = {"ms_per_step": ms, "samples_per_s": B / (ms * 1e-3)}
        del layer, opt, dY, logits
    torch.cuda.empty_cache()
    return out


def cpu_info():
    """The host CPU as /proc/cpuinfo names it (model name, family/model/stepping)
    and how many logical CPUs the host has."""
    fields, n = {}, 0
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k = k.strip()
                if k == "processor":
                    n += 1
                elif k in ("model name", "cpu family", "model", "stepping") and k not in fields:
                    fields[k] = v.strip()
    except OSError:
        return None
    return (f"{fields.get('model name')} (family {fields.get('cpu family')} model "
            f"{fields.get('model')} stepping {fields.get('stepping')}; {n} logical CPUs on the host)")


def cpu_baseline(cfg, budget_s=10.0, max_steps=40):
    """Times the CPU oracle (PyTorch-CPU gather+bmm fwd/bwd + C/OpenMP SR-SGD,
    the reference formulation restated) on the full workload of `cfg` (all
    label groups, no scaling), on every core in this process's affinity: two
    warm-up steps, then steps until `budget_s` seconds of timed work (at least
    3, at most `max_steps`); the median step is reported."""
    import numpy as np
    import torch

    import oracle

    ncores = len(os.sched_getaffinity(0))
    torch.set_num_threads(ncores)
    oracle.set_num_threads(ncores)
    B, D, O, G, F = cfg["B"], cfg["D"], cfg["O"], cfg["G"], cfg["F"]
    Gc = (O + G - 1) // G
    Op = Gc * G  # the oracle works on whole groups; the padding labels are W = 0 columns
    g = torch.Generator().manual_seed(0)
    x = torch.randn(B, D, generator=g).to(torch.bfloat16)
    W = ((torch.rand(Op, F, generator=g) * 2 - 1) / math.sqrt(F)).to(torch.bfloat16)
    W[O:] = 0
    bias = torch.zeros(Op, dtype=torch.bfloat16)
    idx = torch.randint(0, D, (Gc, F), generator=g, dtype=torch.int32)
    dY = (torch.randn(B, Op, generator=g) * 0.1).to(torch.bfloat16)
    dY[:, O:] = 0

    def one_step(seed):
        t = [time.perf_counter()]
        xT = x.t().contiguous()
        oracle.ffi_forward(idx, xT, W, bias, G).to(torch.bfloat16)
        t.append(time.perf_counter())
        dxt = oracle.ffi_backward_features(idx, W, dY, G, D)
        oracle.sr_round_bf16(dxt.t().contiguous().numpy(), 123)
        t.append(time.perf_counter())
        dW = oracle.ffi_backward_weights(idx, xT, dY, G)
        db = oracle.bias_grad(dY)
        t.append(time.perf_counter())
        wb = W.view(torch.int16).numpy().view(np.uint16)
        oracle.sgd_sr_step(wb, dW.numpy(), None, LR, WD, 0.0, False, True, seed)
        oracle.sgd_sr_step(bias.view(torch.int16).numpy().view(np.uint16), db.numpy(), None,
                           LR, WD, 0.0, False, True, seed)
        t.append(time.perf_counter())
        return [b - a for a, b in zip(t, t[1:])]

    one_step(0)  # warm-up
    one_step(0)
    steps = []
    t_start = time.perf_counter()
    while len(steps) < max_steps and (len(steps) < 3 or time.perf_counter() - t_start < budget_s):
        steps.append(one_step(len(steps) + 1))
    timed_s = time.perf_counter() - t_start
    tot = sorted(sum(s) for s in steps)[len(steps) // 2]
    ph = [sorted(s[i] for s in steps)[len(steps) // 2] * 1e3 for i in range(4)]
    return {"value": B / tot, "unit": "samples/s", "cores": ncores, "kind": "port",
            "cpu_model": cpu_info(),
            "sample": (f"oracle (torch-CPU gather+bmm fwd/bwd + C/OpenMP SR-SGD) on the full workload "
                       f"({Gc} label groups, B={B}), median of {len(steps)} steps ({timed_s:.1f} s "
                       f"timed) after 2 warm-ups"),
            "step_ms": round(tot * 1e3, 2),
            "phases_ms": {"fwd": round(ph[0], 2), "bwd_features_sr": round(ph[1], 2),
                          "bwd_weights_dbias": round(ph[2], 2), "sr_sgd": round(ph[3], 2)}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=1, choices=sorted(CONFIGS))
    ap.add_argument("--extra-configs", default="2,3,4",
                    help="comma-separated BASELINE configs also timed (configs 2 and 4 with "
                         "their rewire); '' for none")
    ap.add_argument("--no-dropin", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
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

    dev = torch.device("cuda:0")
    cfg = CONFIGS[args.config]
    B, D, O, G, F = cfg["B"], cfg["D"], cfg["O"], cfg["G"], cfg["F"]
    st, x, dY_buf, pos = setup_step(cfg, dev)
    ldy = st.ldo
    labels = torch.from_numpy(pos).to(dev)  # the same positives as COO (row, label) pairs
    stream = torch.cuda.current_stream()

    ms_per_step, per, wall = timed(step_fns(st, x, dY_buf), args.steps, args.warmup, stream)
    phase_ms = dict(zip(NAMES, per))
    # the same step with separate gradient and SGD kernels (identical results)
    un_names = ["fwd", "bwd_features", "bwd_weights", "sgd"]
    un_ms, un_per, _ = timed([lambda: st.forward(x), lambda: st.backward_features(dY_buf, ldy),
                              lambda: st.backward_weights(dY_buf, ldy), st.sgd],
                             max(5, args.steps // 2), 2, stream)
    # the step with the loss fused into the forward (dY from the labels; the logits
    # are not written): what a training loop runs per batch
    fl_names = ["fwd_bce", "bwd_features", "bwd_weights_sgd"]
    fl_ms, fl_per, _ = timed([lambda: st.forward_bce(x, labels),
                              lambda: st.backward_features(st.dY_buf, ldy, defer_dx=True),
                              lambda: st.backward_weights_sgd(st.dY_buf, ldy)],
                             max(5, args.steps // 2), 2, stream)

    # the same fused step captured once in a HIP graph and replayed (the SR-SGD seed
    # read and advanced on the device), on a copy of the parameters
    from haste_amd.step import FFITrainStep
    gst = FFITrainStep(st.W.clone(), None if st.bias is None else st.bias.clone(), st.idx, B, D,
                       G, lr=LR, weight_decay=WD, seed=SEED, device_seed=True)
    gst.step(x, dY_buf, ldy)   # builds the index plan outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gst.step(x, dY_buf, ldy)
    gr_ms, _, _ = timed([graph.replay], max(5, args.steps // 2), 2, stream)
    del graph, gst

    word_rate = sr_word_rate(dev)
    pb = phase_bytes(B, D, O, G, F)
    phase_gbs = {n: pb[n] / (phase_ms[n] * 1e-3) / 1e9 for n in NAMES}
    dom = max(NAMES, key=lambda n: phase_ms[n])
    rep = phase_report(cfg, ms_per_step, per)
    result = {
        "metric": METRIC,
        "value": B / (ms_per_step * 1e-3),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_min_ms": WARM_MS,
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
        "step_roofline": {"bytes": sum(pb[n] for n in NAMES), "hbm_frac": rep["step_hbm_frac"],
                          "mfma_frac": rep["step_mfma_frac"]},
        "phases_us": rep["phases_us"],
        "phases_hbm_frac": rep["phases_hbm_frac"],
        "sr_floor": {"words_per_s": word_rate,
                     "probe": "haste_sr_words_fold: 2^26 tl.randint words, XOR-folded 64 to 1",
                     "phases": sr_floor_report(cfg, dict(phase_ms, sgd=un_per[3]), word_rate)},
        "unfused": {"ms_per_step": un_ms, "samples_per_s": B / (un_ms * 1e-3),
                    "phases_us": {n: round(v * 1e3, 2) for n, v in zip(un_names, un_per)}},
        "fused_loss": {"ms_per_step": fl_ms, "samples_per_s": B / (fl_ms * 1e-3),
                       "phases_us": {n: round(v * 1e3, 2) for n, v in zip(fl_names, fl_per)},
                       "workload": "forward + sparse BCE gradient from COO labels (loss summed "
                                   "on the device, logits not written) + bwd_features + "
                                   "bwd_weights + SR-SGD"},
        "hip_graph": {"ms_per_step": gr_ms, "samples_per_s": B / (gr_ms * 1e-3),
                      "workload": "the same step captured once in a HIP graph "
                                  "(FFITrainStep(device_seed=True)) and replayed"},
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
            # an elementwise kernel (torch's own copy_ is a runtime blit, whose
            # writes WRITE_SIZE has not always counted)
            torch.mul(src, 1.0, out=dst)
        torch.cuda.synchronize()
        del src, dst
    del st, x, dY_buf, labels
    torch.cuda.empty_cache()
    if not args.no_dropin:
        d = time_dropin(cfg, max(10, args.steps // 2), 3, dev)
        for v in d.values():
            v["vs_train_step"] = round(v["ms_per_step"] / ms_per_step, 3)
        result["dropin_api"] = dict(d, workload="GroupFixedFanIn forward (x requires grad) + "
                                    "autograd backward of a [B, O] grad + SRSgd.step (momentum 0)")
    extras = [int(c) for c in args.extra_configs.split(",") if c.strip()]
    if extras:
        result["configs"] = {str(c): run_extra_config(c, max(10, args.steps // 2), 3, dev,
                                                      word_rate)
                             for c in extras if c != args.config}
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(cfg)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
