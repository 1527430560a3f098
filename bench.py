#!/usr/bin/env python3
"""Fold throughput of the HardShell hot path on one MI355X.

Default workload: a GPT-2-small-shape integer model in .hsm layout (12 layers, d_model 768,
12 heads x 64, d_ff 3072, vocab 50,257, n_ctx 1,024) with seeded uniform int8 weights, folding
a 16,384-token Zipf(1.1) stream as 64 independent 256-token windows (blocks of 1,024 bytes of
fixed-width 4-byte tokens) batched on one GPU. One step is one whole fold: the integer forward
pass of all 16,384 rows, the logits -> CDF coder op on the GPU, the host range coder, the block
payloads and the .taco container. Four batches are in flight by default (--batches; fewer when
they would not fit in three quarters of the device memory): each folds
whole steps from its own host thread on its own stream, so one batch's host work and kernels
overlap the others' kernels; every step's container must equal the first one's. `one_batch`
is the same steps on a single batch (its wall time, the GPU span of its passes, the host's
share). The warmup steps run one batch at a time (each batch's first use), then again with the
batches in flight right before the timed ones.

Prints one JSON line. `value` is fold tokens per second with the token stream and the model
already resident (model upload and token staging are outside the timed region; per step the
host sends 8 B and receives 24 B per token). `roofline` is the int8 GEMM kernels against the
MI355X dense int8 MFMA peak, from hipEvents around every launch on the batch stream in as many
profiled steps, run right after the timed ones (events around every launch leave the GPU idle
about 10 us between kernels, so the timed steps run without them).
`cpu_baseline` is the oracle's C++ restatement of the reference CPU fast path (AVX2 products,
prefill chunk 32, one window per thread) timed on a sample of the same windows in the same run,
on every core the process may use within the GPU's CPU share (OMP_NUM_THREADS when set; the
CPU model and core counts are recorded) and (`one_thread`) on one thread over the first window;
its payloads must equal the GPU's. `sustained` is the same fold repeated for at least 3 s right
after the timed steps.

Other workloads (--workload) measure the other configurations of the path, each with its own
line: the c_attn GEMM alone (gemm-qkv: M 256 and 16,384, K 768, N 2,304), decode attention over
HBM-resident caches (attend-decode: 64 streams x 12 heads x 64, contexts 128 / 512 / 1,024),
the GPT-2-medium fold with the full unfold round trip (fold-gpt2-medium: 256 x 256 tokens),
the GPT-2-XL fold (fold-gpt2-xl: 512 x 512 tokens), and the fold's GEMM shapes beside the vendor
library's int8 product (gemm-vendor: hipBLASLt through torch._int_mm, i32 outputs, no epilogue).
"""

import argparse
import ctypes as C
import hashlib
import json
import os
import sys
import threading
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA, 5.0 POPS
HBM_PEAK_GBS = 8000.0

FOLDS = {  # workload -> (dims name, windows, tokens per window, CPU-baseline windows per thread)
    "fold-gpt2-small": ("GPT2_SMALL", 64, 256, 4),
    "fold-gpt2-medium": ("GPT2_MEDIUM", 256, 256, 2),
    "fold-gpt2-xl": ("GPT2_XL", 512, 512, 1),
}


def log(msg):
    print(msg, file=sys.stderr, flush=True)


HERE = os.path.dirname(os.path.abspath(__file__))


def traffic_summary(fetch_csv, write_csv, calib_mib, tokens_sha, command):
    """HBM bytes per dispatch of each kernel from two rocprofv3 --pmc runs (FETCH_SIZE, then
    WRITE_SIZE, KiB per dispatch). Each counter is scaled by what it reads for the calibration
    copy of calib_mib MiB (the largest __amd_rocclr_copyBuffer dispatch of the run)."""
    import csv
    import collections

    def load(path):
        per = collections.defaultdict(float)
        for r in csv.DictReader(open(path)):
            name = r["Kernel_Name"].split("(")[0].replace("void ", "").strip()
            per[(name, r["Dispatch_Id"])] += float(r["Counter_Value"])
        return per

    fetch, write = load(fetch_csv), load(write_csv)
    copy_kib = calib_mib * 1024.0
    f_copy = max(v for (k, _), v in fetch.items() if "copyBuffer" in k)
    w_copy = max(v for (k, _), v in write.items() if "copyBuffer" in k)
    f_scale, w_scale = copy_kib / f_copy, copy_kib / w_copy
    agg = collections.defaultdict(lambda: [0, 0.0, 0.0])
    for (k, d), v in fetch.items():
        if "rocclr" in k:
            continue
        agg[k][0] += 1
        agg[k][1] += v * f_scale * 1024
    for (k, d), v in write.items():
        if "rocclr" in k:
            continue
        agg[k][2] += v * w_scale * 1024
    return {"library": library_version(), "tokens_sha256": tokens_sha, "command": command,
            "calibration_mib": calib_mib,
            "fetch_scale": round(f_scale, 4), "write_scale": round(w_scale, 4),
            "kernels": {k: {"dispatches": n, "fetch_bytes": round(fb / n), "write_bytes": round(wb / n)}
                        for k, (n, fb, wb) in sorted(agg.items())}}


def calibration_copy(hip, dev, mib):
    """One device-to-device copy of mib MiB: the counter runs scale FETCH_SIZE and WRITE_SIZE by
    what they read for it."""
    nb = mib << 20
    src, dst = C.c_void_p(), C.c_void_p()
    hip._check(hip.lib().hs_device_alloc(dev.h, nb, C.byref(src)))
    hip._check(hip.lib().hs_device_alloc(dev.h, nb, C.byref(dst)))
    hip._check(hip.lib().hs_device_copy(dev.h, dst, src, nb))
    hip.lib().hs_device_free(dev.h, src)
    hip.lib().hs_device_free(dev.h, dst)
    log(f"calibration copy: {mib} MiB device to device")


ATTEND_CONTEXTS = ((128, 64), (512, 16), (1024, 8))  # (ctx, cache sets): two launches per set


def attend_traffic_summary(fetch_csv, write_csv, calib_mib, command):
    """HBM bytes per decode-attention launch at each context of the attend-decode workload, from
    two rocprofv3 --pmc runs (FETCH_SIZE, then WRITE_SIZE), scaled by the calibration copy. The
    workload launches 2 * sets decode-attention kernels per context, contexts in order (the wave
    per row-head form up to 256 keys, the one-launch form above)."""
    import csv
    import collections

    def load(path):
        per = collections.defaultdict(float)
        for r in csv.DictReader(open(path)):
            per[(r["Kernel_Name"], int(r["Dispatch_Id"]))] += float(r["Counter_Value"])
        return per

    fetch, write = load(fetch_csv), load(write_csv)
    copy_kib = calib_mib * 1024.0
    f_scale = copy_kib / max(v for (k, _), v in fetch.items() if "copyBuffer" in k)
    w_scale = copy_kib / max(v for (k, _), v in write.items() if "copyBuffer" in k)
    def attn(per):  # the decode-attention dispatches in launch order
        return [(k, v) for (k, d), v in sorted(per.items(), key=lambda kv: kv[0][1])
                if "k_attend_decode" in k or "k_split_pv" in k]

    fd, wd = attn(fetch), attn(write)
    out = {}
    if len(fd) == sum(2 * sets for _, sets in ATTEND_CONTEXTS) and len(wd) == len(fd):
        i = 0
        for ctx, sets in ATTEND_CONTEXTS:
            n = 2 * sets
            out[str(ctx)] = {"kernel": fd[i][0].split("(")[0].replace("void ", ""), "dispatches": n,
                             "algorithmic_bytes": 2 * 64 * 12 * ctx * 64 + 2 * 64 * 12 * 64,
                             "fetch_bytes": round(sum(v for _, v in fd[i:i + n]) / n * f_scale * 1024),
                             "write_bytes": round(sum(v for _, v in wd[i:i + n]) / n * w_scale * 1024)}
            i += n
    return {"library": library_version(), "command": command, "calibration_mib": calib_mib,
            "fetch_scale": round(f_scale, 4), "write_scale": round(w_scale, 4), "contexts": out}


def library_version():
    """hs_version() of the loaded library: the SHA-256 prefix of the kernel sources it was built
    from. Counter summaries record it, and a summary of another build is not reported."""
    from taco_amd import hip
    return hip.version()


def _same_build(summary):
    return summary.get("library") == library_version()


def committed_attend_traffic(ctx):
    """HBM bytes per decode-attention launch at ctx from the committed summary of this build, or
    None."""
    path = os.path.join(HERE, "profiles", "attend_decode_traffic.json")
    if not os.path.exists(path):
        return None
    j = json.load(open(path))
    if not _same_build(j):
        return None
    c = j.get("contexts", {}).get(str(ctx))
    return c["fetch_bytes"] + c["write_bytes"] if c else None


def committed_traffic(workload, tokens_sha):
    """The GEMM HBM bytes per launch of the committed traffic summary of this workload (the same
    token stream), or None."""
    path = os.path.join(HERE, "profiles", workload.replace("-", "_") + "_traffic.json")
    if not os.path.exists(path):
        return None
    t = json.load(open(path))
    if t.get("tokens_sha256") != tokens_sha or not _same_build(t):
        return None
    g = [v for k, v in t["kernels"].items() if "k_gemm" in k]
    n = sum(v["dispatches"] for v in g)
    if n == 0:
        return None
    return round(sum((v["fetch_bytes"] + v["write_bytes"]) * v["dispatches"] for v in g) / n)


def mfma_summary(csv_path, tokens_sha, command):
    """Per-kernel MFMA utilisation from one rocprofv3 --pmc run of SQ_INSTS_VALU_MFMA_MOPS_I8,
    SQ_VALU_MFMA_BUSY_CYCLES, GRBM_GUI_ACTIVE and SQ_BUSY_CYCLES: MfmaUtil = busy cycles /
    (GUI-active cycles of one XCD x 1,024 SIMDs), as rocprofv3's derived counter; int8 ops =
    MOPS_I8 x 512 (the counter counts ops / 512)."""
    import csv
    import collections
    per = collections.defaultdict(dict)
    for r in csv.DictReader(open(csv_path)):
        k = (int(r["Dispatch_Id"]), r["Kernel_Name"])
        per[k][r["Counter_Name"]] = float(r["Counter_Value"])
    agg = collections.defaultdict(lambda: collections.defaultdict(float))
    for (_, name), c in per.items():
        if not c.get("SQ_INSTS_VALU_MFMA_MOPS_I8"):
            continue
        a = agg[name.split("(")[0].replace("void ", "")]
        a["dispatches"] += 1
        for kk, v in c.items():
            a[kk] += v
    kernels, tot_busy, tot_gui, tot_ops = {}, 0.0, 0.0, 0.0
    for name, a in sorted(agg.items()):
        gui1 = a["GRBM_GUI_ACTIVE"] / 8  # GRBM_GUI_ACTIVE summed over the 8 XCDs
        kernels[name] = {"dispatches": int(a["dispatches"]),
                         "mfma_util": round(a["SQ_VALU_MFMA_BUSY_CYCLES"] / (gui1 * 1024), 4),
                         "int8_ops_per_dispatch": int(a["SQ_INSTS_VALU_MFMA_MOPS_I8"] * 512 / a["dispatches"]),
                         "gui_cycles_per_dispatch": int(gui1 / a["dispatches"])}
        if name.startswith("hs::k_gemm"):
            tot_busy += a["SQ_VALU_MFMA_BUSY_CYCLES"]
            tot_gui += gui1 * 1024
            tot_ops += a["SQ_INSTS_VALU_MFMA_MOPS_I8"] * 512
    return {"library": library_version(), "tokens_sha256": tokens_sha, "command": command,
            "gemm_mfma_util": round(tot_busy / tot_gui, 4) if tot_gui else None,
            "gemm_int8_ops": int(tot_ops), "kernels": kernels}


SQ_PASSES = (
    ("SQ_WAVES", "SQ_INSTS_VALU", "SQ_INSTS_SALU", "SQ_INSTS_LDS", "SQ_INSTS_MFMA",
     "SQ_INSTS_VMEM_RD", "SQ_INSTS_VMEM_WR", "SQ_WAVE_CYCLES"),
    ("SQ_WAVE_CYCLES", "SQ_ACTIVE_INST_VALU", "SQ_ACTIVE_INST_LDS", "SQ_WAIT_INST_ANY",
     "SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE", "SQ_BUSY_CYCLES", "GRBM_GUI_ACTIVE"),
)


def sq_summary(csv_paths, tokens_sha, command):
    """Per-kernel instruction mix from the two rocprofv3 --pmc runs of SQ_PASSES: instructions
    per wave by kind, and, as fractions of the waves' lifetime (SQ_WAVE_CYCLES, quad-cycles like
    the ACTIVE and WAIT counters), the cycles spent issuing VALU and LDS instructions and waiting
    to issue; LDS bank-conflict cycles per LDS-active cycle."""
    import csv
    import collections
    agg = collections.defaultdict(lambda: collections.defaultdict(float))
    for pi, path in enumerate(csv_paths):
        per = collections.defaultdict(dict)
        for r in csv.DictReader(open(path)):
            per[(int(r["Dispatch_Id"]), r["Kernel_Name"])][r["Counter_Name"]] = float(r["Counter_Value"])
        for (_, name), c in per.items():
            a = agg[name.split("(")[0].replace("void ", "")]
            a[f"dispatches{pi}"] += 1
            for kk, v in c.items():
                a[f"{kk}#{pi}"] += v
    kernels = {}
    for name, a in sorted(agg.items()):
        n0, n1 = a["dispatches0"], a["dispatches1"]
        if not n0 or not n1 or not a["SQ_WAVES#0"]:
            continue
        waves = a["SQ_WAVES#0"] / n0
        per_wave = lambda k: round(a[k + "#0"] / n0 / waves, 1)
        wc = a["SQ_WAVE_CYCLES#1"]
        kernels[name] = {
            "dispatches": int(n0), "waves_per_dispatch": int(waves),
            "valu_per_wave": per_wave("SQ_INSTS_VALU"), "salu_per_wave": per_wave("SQ_INSTS_SALU"),
            "lds_per_wave": per_wave("SQ_INSTS_LDS"), "mfma_per_wave": per_wave("SQ_INSTS_MFMA"),
            "vmem_rd_per_wave": per_wave("SQ_INSTS_VMEM_RD"), "vmem_wr_per_wave": per_wave("SQ_INSTS_VMEM_WR"),
            "valu_active_frac": round(a["SQ_ACTIVE_INST_VALU#1"] / wc, 3) if wc else None,
            "lds_active_frac": round(a["SQ_ACTIVE_INST_LDS#1"] / wc, 3) if wc else None,
            "wait_frac": round(a["SQ_WAIT_INST_ANY#1"] / wc, 3) if wc else None,
            "lds_conflict_per_active": (round(a["SQ_LDS_BANK_CONFLICT#1"] / a["SQ_LDS_IDX_ACTIVE#1"], 3)
                                        if a["SQ_LDS_IDX_ACTIVE#1"] else None),
            "gui_cycles_per_dispatch": int(a["GRBM_GUI_ACTIVE#1"] / 8 / n1)}
    return {"library": library_version(), "tokens_sha256": tokens_sha, "command": command, "kernels": kernels}


def committed_mfma(workload, tokens_sha):
    """The GEMM MFMA utilisation of the committed counter summary of this workload, or None."""
    path = os.path.join(HERE, "profiles", workload.replace("-", "_") + "_mfma.json")
    if not os.path.exists(path):
        return None
    j = json.load(open(path))
    return j["gemm_mfma_util"] if j.get("tokens_sha256") == tokens_sha and _same_build(j) else None


def host_cpu():
    """The host's CPU model, online cores and the cores this process may run on."""
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"cpu_model": model, "nproc": os.cpu_count(),
            "affinity": len(os.sched_getaffinity(0))}


def read_profile(hip, batch):
    cap = 32
    labels = C.create_string_buffer(32 * cap)
    ns = np.zeros(cap, np.uint64)
    launches = np.zeros(cap, np.uint64)
    ops = np.zeros(cap, np.uint64)
    k = hip.lib().hs_batch_profile(batch.h, labels, ns.ctypes.data_as(C.c_void_p),
                                   launches.ctypes.data_as(C.c_void_p),
                                   ops.ctypes.data_as(C.c_void_p), cap, 1)
    prof = {}
    for i in range(k):
        name = labels.raw[32 * i:32 * i + 32].split(b"\0")[0].decode()
        prof[name] = dict(ns=int(ns[i]), launches=int(launches[i]), ops=int(ops[i]))
    return prof


def run_fold(args):
    from taco_amd import fold, hip, synth
    dims_name, W, n, cpu_per_thread = FOLDS[args.workload]
    if args.windows:
        W = args.windows
    if args.window_tokens:
        n = args.window_tokens
    dims = getattr(synth, dims_name)
    t0 = time.time()
    log(f"building the {dims_name} model and {W} x {n} tokens")
    model_bytes = synth.build_model(dims)
    tokens = synth.zipf_tokens(W * n)
    blocks = [tokens[w * n:(w + 1) * n] for w in range(W)]
    original = fold.token_bytes(tokens)
    block_size = 4 * n
    log(f"workload built in {time.time() - t0:.1f}s: model {len(model_bytes)} B "
        f"sha256 {hashlib.sha256(model_bytes).hexdigest()[:16]}, tokens sha256 "
        f"{synth.sha256_tokens(tokens)[:16]}")

    dev = hip.HipDevice.open(0)
    if args.calib_copy_mib:
        calibration_copy(hip, dev, args.calib_copy_mib)
    model = hip.HipModel.load(dev, model_bytes)
    # Batches in flight: each folds whole steps from its own host thread on its own stream, so
    # one batch's host work (plan, inputs, range coding, container) and kernels overlap the
    # other's kernels. The first batch also runs the one-batch, profiled and unfold parts.
    # The batches beyond the first are made while they fit in three quarters of the device
    # memory left (the GPT-2-XL workload's caches take about 80 GB per batch).
    batches = [hip.HipBatch(model, W, W * n)]
    per_batch = batches[0].gpu_bytes()
    while len(batches) < max(1, args.batches) and per_batch <= 0.75 * dev.memory()[0]:
        batches.append(hip.HipBatch(model, W, W * n))
    nb = len(batches)
    batch = batches[0]
    log(f"device {dev.name()}, model {model.weight_bytes() / 1e6:.1f} MB, {nb} batch(es) of "
        f"{batch.gpu_bytes() / 1e9:.2f} GB")

    phase = {"fold": 0.0, "container": 0.0}

    def step(b=None):
        t0 = time.perf_counter()
        payloads = fold.fold_blocks(b or batch, blocks, 0)  # every row runs (no early stop)
        t1 = time.perf_counter()
        cont = fold.container(model.hash(), original, block_size, 0, payloads)
        phase["fold"] += t1 - t0
        phase["container"] += time.perf_counter() - t1
        return payloads, cont

    def steps_in_flight(k):
        """k steps over the batches, batch t taking steps t, t + nb, ... on its own thread;
        returns the wall time and every step's container."""
        conts, errors = [[] for _ in range(nb)], []

        def run(t):
            try:
                for _ in range(t, k, nb):
                    conts[t].append(step(batches[t])[1])
            except Exception as e:  # surfaced on the main thread
                errors.append(e)

        threads = [threading.Thread(target=run, args=(t,)) for t in range(nb)]
        t0 = time.perf_counter()
        for th in threads:
            th.start()
        for th in threads:
            th.join()
        el = time.perf_counter() - t0
        if errors:
            raise errors[0]
        return el, [c for cs in conts for c in cs]

    for i in range(max(args.warmup, nb)):
        ts = time.time()
        payloads, cont = step(batches[i % nb])
        log(f"warmup {i}: {time.time() - ts:.3f}s, container {len(cont)} B")
    # The timed steps run without per-launch events (an event pair around every launch costs
    # about 10 us of idle GPU between kernels); the per-op times and the roofline come from the
    # same number of profiled steps right after them.
    # The timed steps record one event pair per forward pass (no per-launch events): the GPU
    # span of the passes, so the host's share of a step is the wall time minus the span.
    # One batch alone first: its wall time, the GPU span of its passes (one event pair per
    # pass) and so the host's share of a step.
    phase.update(fold=0.0, container=0.0)
    hip._check(hip.lib().hs_batch_set_profiling(batch.h, 2))
    hip.lib().hs_batch_profile(batch.h, None, None, None, None, 0, 1)
    ts = time.perf_counter()
    for i in range(args.steps):
        payloads, cont = step()
    one_elapsed = time.perf_counter() - ts
    span = read_profile(hip, batch).get("pass_span", {"ns": 0, "launches": 0})
    hip._check(hip.lib().hs_batch_set_profiling(batch.h, 0))
    span_ms = span["ns"] / 1e6 / max(1, args.steps)
    host_ms = 1e3 * one_elapsed / max(1, args.steps) - span_ms
    log(f"one batch: {1e3 * one_elapsed / args.steps:.3f} ms per step; GPU span of the passes "
        f"{span_ms:.3f} ms per step ({span['launches']} passes), host share {host_ms:.3f} ms per step")
    timed_phase = dict(phase)
    # The warmup steps again, now with the batches in flight (the steps above ran one batch
    # alone), so the timed region starts with every batch's thread and stream already busy.
    steps_in_flight(max(args.warmup, nb))
    # The timed steps: the batches in flight
    elapsed, conts = steps_in_flight(args.steps)
    if any(c != cont for c in conts):
        log("PARITY FAILURE: a batch in flight gave another container")
        sys.exit(1)
    log(f"timed: {args.steps} steps on {nb} batch(es) in flight: {1e3 * elapsed / args.steps:.3f} ms per step")
    # Sustained: fold steps for at least args.sustain_s seconds right after the timed ones (the
    # timed region is short enough to end before the clocks settle under a sustained MFMA load).
    sustained = None
    if args.sustain_s > 0:
        ss, s_el = 0, 0.0
        while s_el < args.sustain_s:
            el, sconts = steps_in_flight(4 * nb)
            ss += len(sconts)
            s_el += el
            if any(c != cont for c in sconts):
                log("PARITY FAILURE: the sustained steps gave another container")
                sys.exit(1)
        sustained = {"seconds": round(s_el, 3), "steps": ss,
                     "tokens_per_s": round(W * n * ss / s_el, 1),
                     "ms_per_step": round(1e3 * s_el / ss, 3)}
        log(f"sustained: {ss} steps in {s_el:.2f}s -> {W * n * ss / s_el:.0f} tokens/s")
    psteps = max(1, args.steps)
    hip._check(hip.lib().hs_batch_set_profiling(batch.h, 1))
    hip.lib().hs_batch_profile(batch.h, None, None, None, None, 0, 1)
    tp = time.perf_counter()
    for i in range(psteps):
        ppay, pcont = step()
    profiled_s = time.perf_counter() - tp
    hip._check(hip.lib().hs_batch_set_profiling(batch.h, 0))
    prof = read_profile(hip, batch)
    if pcont != cont:
        log("PARITY FAILURE: the profiled steps gave another container")
        sys.exit(1)
    gemm = [v for kk, v in prof.items() if kk.startswith("gemm")]
    gemm_ns = sum(v["ns"] for v in gemm)
    gemm_ops = sum(v["ops"] for v in gemm)
    gemm_launches = sum(v["launches"] for v in gemm)
    achieved = gemm_ops / gemm_ns / 1e3 if gemm_ns else 0.0  # ops/ns -> TOPS
    tokens_per_step = W * n
    value = tokens_per_step * args.steps / elapsed
    cont_sha = hashlib.sha256(cont).hexdigest()
    coded = sum(1 for p in payloads if p is not None and len(p) < block_size)
    log(f"timed: {args.steps} steps in {elapsed:.3f}s -> {value:.0f} tokens/s; container "
        f"{len(cont)} B sha256 {cont_sha[:16]}, {coded}/{W} blocks coded")
    gpu_ms = sum(v["ns"] for v in prof.values()) / 1e6 / psteps
    log(f"  per step: fold call {1e3 * timed_phase['fold'] / args.steps:.3f} ms, container "
        f"{1e3 * timed_phase['container'] / args.steps:.3f} ms; profiled steps "
        f"{1e3 * profiled_s / psteps:.3f} ms (kernels {gpu_ms:.3f} ms)")
    for kk, v in sorted(prof.items(), key=lambda x: -x[1]["ns"]):
        log(f"  {kk:12s} {v['ns'] / 1e6 / psteps:8.3f} ms/step  {v['launches'] // psteps:5d} "
            f"launches/step" + (f"  {v['ops'] / v['ns'] / 1e3:7.1f} TOPS" if v["ops"] and v["ns"] else ""))

    unfold = None
    if args.workload == "fold-gpt2-medium" and not args.no_unfold:
        # the full round trip: every block decoded on the GPU (one row per slot per call), with
        # one event pair per pass (the GPU span of the passes, gaps between kernels included)
        hip._check(hip.lib().hs_batch_set_profiling(batch.h, 2))
        hip.lib().hs_batch_profile(batch.h, None, None, None, None, 0, 1)
        ts = time.perf_counter()
        back = fold.unfold_blocks(batch, payloads, 0, cap=n)
        u_s = time.perf_counter() - ts
        uspan = read_profile(hip, batch).get("pass_span", {"ns": 0, "launches": 0})
        hip._check(hip.lib().hs_batch_set_profiling(batch.h, 0))
        same = all(np.array_equal(back[w], blocks[w]) for w in range(W))
        log(f"unfold: {W} blocks in {u_s:.3f}s -> {W * n / u_s:.0f} tokens/s; round trip equal: {same}")
        if not same:
            log("ROUND TRIP FAILURE: the unfolded tokens differ")
            sys.exit(1)
        # the same round trip again with an event pair around every launch: GPU time per op
        # for each decode pass (one row per slot), against the wall time of the timed run
        hip._check(hip.lib().hs_batch_set_profiling(batch.h, 1))
        hip.lib().hs_batch_profile(batch.h, None, None, None, None, 0, 1)
        back2 = fold.unfold_blocks(batch, payloads, 0, cap=n)
        hip._check(hip.lib().hs_batch_set_profiling(batch.h, 0))
        uprof = read_profile(hip, batch)
        if not all(np.array_equal(back2[w], blocks[w]) for w in range(W)):
            log("ROUND TRIP FAILURE: the profiled unfold differs")
            sys.exit(1)
        passes = max(v["launches"] for kk, v in uprof.items() if kk == "embed")
        u_ops = {kk: round(v["ns"] / 1e6 / passes, 4) for kk, v in sorted(uprof.items(), key=lambda x: -x[1]["ns"])}
        log(f"unfold: {passes} passes; GPU ms per pass by op: {u_ops}; wall ms per pass "
            f"{1e3 * u_s / passes:.3f}")
        span_pass = uspan["ns"] / 1e6 / max(1, uspan["launches"])
        log(f"unfold: GPU span {span_pass:.3f} ms per pass over {uspan['launches']} passes; wall "
            f"{1e3 * u_s / max(1, uspan['launches']):.3f} ms per pass")
        unfold = {"tokens_per_s": round(W * n / u_s, 1), "seconds": round(u_s, 3),
                  "round_trip_equal": same, "passes": passes,
                  "wall_ms_per_pass": round(1e3 * u_s / passes, 4),
                  "gpu_span_ms_per_pass": round(span_pass, 4),
                  "gpu_ms_per_pass_by_op": u_ops}

    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O
        # every core this process may run on, within the GPU's CPU share when the environment
        # states one (OMP_NUM_THREADS)
        host = host_cpu()
        share = int(os.environ.get("OMP_NUM_THREADS") or host["affinity"])
        threads = args.cpu_threads or max(1, min(host["affinity"], share))
        cw = min(args.cpu_windows or cpu_per_thread * threads, W)
        om = O.Model(model_bytes)
        ts = time.perf_counter()
        cpu_payloads = O.fold_payloads(om, tokens[:cw * n], cw, n, chunk=32, threads=threads)
        cpu_s = time.perf_counter() - ts
        same = all(cpu_payloads[w] == payloads[w] for w in range(cw))
        log(f"cpu baseline: {cw} windows x {n} tokens on {threads} threads in {cpu_s:.2f}s; "
            f"payloads equal to the GPU's: {same}")
        if not same:
            log("PARITY FAILURE: the CPU and GPU payloads differ")
            sys.exit(1)
        # the same restatement on one thread, over the first window
        ts = time.perf_counter()
        one = O.fold_payloads(om, tokens[:n], 1, n, chunk=32, threads=1)
        one_s = time.perf_counter() - ts
        same1 = one[0] == payloads[0]
        log(f"cpu baseline, one thread: 1 window x {n} tokens in {one_s:.2f}s; payload equal to the GPU's: {same1}")
        if not same1:
            log("PARITY FAILURE: the one-thread CPU payload differs")
            sys.exit(1)
        cpu = {"value": round(cw * n / cpu_s, 2), "unit": "tokens/s", "cores": threads,
               "kind": "port", "host": dict(host, cpu_share=share),
               "sample": f"the first {cw} of the {W} windows ({cw * n} tokens), {cpu_per_thread} "
                         f"window(s) per thread, AVX2 restatement of the reference CPU fast path, "
                         f"chunk 32",
               "payloads_equal_gpu": same,
               "one_thread": {"value": round(n / one_s, 2), "unit": "tokens/s", "cores": 1,
                              "sample": f"the first window ({n} tokens)", "payload_equal_gpu": same1}}

    label = {"fold-gpt2-small": "GPT-2 124M", "fold-gpt2-medium": "GPT-2 medium 355M",
             "fold-gpt2-xl": "GPT-2 XL 1.5B"}[args.workload]
    out = {
        "metric": f"fold tokens/sec on 1 MI355X ({label} int8, bit-exact); int8 MFMA % of peak",
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * elapsed / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": f"{dims_name.lower().replace('_', '-')}-shape fold: {W} windows x "
                               f"{n} Zipf(1.1) tokens",
                   "layers": dims.n_layer, "d_model": dims.d_model, "heads": dims.n_head,
                   "d_ff": dims.d_ff, "vocab": dims.vocab, "n_ctx": dims.n_ctx,
                   "tokens_per_step": tokens_per_step, "batches_in_flight": nb,
                   "container_sha256": cont_sha,
                   "tokens_sha256": synth.sha256_tokens(tokens)},
        "roofline": {"bound": "mfma", "kernel": "k_gemm (all int8 GEMMs of the pass)",
                     "achieved": round(achieved, 2), "peak": INT8_PEAK_TOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / INT8_PEAK_TOPS, 4),
                     "traffic": committed_traffic(args.workload, synth.sha256_tokens(tokens)),
                     "traffic_unit": "HBM bytes per launch (FETCH_SIZE + WRITE_SIZE, calibrated; "
                                     "profiles/" + args.workload.replace("-", "_") + "_traffic.json)",
                     "mfma_util": committed_mfma(args.workload, synth.sha256_tokens(tokens)),
                     "mfma_util_source": "SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE x 1,024 "
                                         "SIMDs) over the GEMM dispatches; profiles/" +
                                         args.workload.replace("-", "_") + "_mfma.json",
                     "launches": gemm_launches,
                     "ops_per_launch": gemm_ops // max(1, gemm_launches),
                     "avg_launch_us": round(gemm_ns / max(1, gemm_launches) / 1e3, 2)},
        "ops_ms_per_step": {kk: round(v["ns"] / 1e6 / psteps, 3) for kk, v in prof.items()},
        "profiled_steps": {"steps": psteps, "ms_per_step": round(1e3 * profiled_s / psteps, 3),
                           "kernel_ms_per_step": round(gpu_ms, 3)},
        "one_batch": {"ms_per_step": round(1e3 * one_elapsed / args.steps, 3),
                      "tokens_per_s": round(tokens_per_step * args.steps / one_elapsed, 1),
                      "gpu_span_ms_per_step": round(span_ms, 3),
                      "host_ms_per_step": round(host_ms, 3)},
        "gpu_span_ms_per_step": round(span_ms, 3),
        "host_ms_per_step": round(host_ms, 3),
        "sustained": sustained,
        "cpu_baseline": cpu,
    }
    if unfold:
        out["unfold"] = unfold
    print(json.dumps(out), flush=True)


def _dev_buf(hip, dev, arr):
    p = C.c_void_p()
    hip._check(hip.lib().hs_device_alloc(dev.h, arr.nbytes, C.byref(p)))
    hip._check(hip.lib().hs_device_upload(dev.h, p, arr.ctypes.data_as(C.c_void_p), arr.nbytes))
    return p


def run_gemm(args):
    """The c_attn linear alone (i8 x i8 -> i32, bias, per-channel rescale, clamp to +-127):
    K 768, N 2,304 at M 256 (one decode batch) and M 16,384 (the fold pass)."""
    from oracle import oracle as O
    from taco_amd import hip
    dev = hip.HipDevice.open(0)
    rng = np.random.default_rng(0xC1)
    K, N, shift = 768, 2304, 42
    w = rng.integers(-127, 128, (N, K)).astype(np.int8)
    bias = rng.integers(-(1 << 16), (1 << 16) + 1, N).astype(np.int32)
    mult = rng.integers(1 << 30, 1 << 31, N).astype(np.int64).astype(np.int32)
    results = []
    for M, reps in ((256, 2000), (16384, 50)):
        a = rng.integers(-127, 128, (M, K)).astype(np.int8)
        mp, np_, kp = hip.gemm_layout(M, N, K)
        wp, ap = hip.gemm_pack(w, np_, kp), hip.gemm_pack(a, mp, kp)
        bufs = [_dev_buf(hip, dev, x) for x in (wp, ap, bias, mult)]
        out = np.zeros((M, N), np.int8)
        dout = _dev_buf(hip, dev, out)
        ns = C.c_uint64()
        hip._check(hip.lib().hs_op_gemm_requant_gpu_ns(dev.h, bufs[0], bufs[1], bufs[2], bufs[3],
                                                         shift, M, N, K, dout, 10, C.byref(ns)))
        hip._check(hip.lib().hs_op_gemm_requant_gpu_ns(dev.h, bufs[0], bufs[1], bufs[2], bufs[3],
                                                         shift, M, N, K, dout, reps, C.byref(ns)))
        hip._check(hip.lib().hs_device_download(dev.h, out.ctypes.data_as(C.c_void_p), dout,
                                                out.nbytes))
        for p in bufs + [dout]:
            hip.lib().hs_device_free(dev.h, p)
        us = ns.value / reps / 1e3
        ops = 2 * M * N * K
        rows = min(M, 256)  # the oracle's rows (the first 256)
        want = O.linear_act_ref(w, a[:rows], bias, mult, shift)
        same = bool(np.array_equal(out[:rows], want))
        ts = time.perf_counter()
        O.matmul_i8(w, a[:rows])
        cpu_s = time.perf_counter() - ts
        log(f"gemm M {M}: {us:.2f} us per launch, {ops / us / 1e6:.1f} TOPS, "
            f"rows 0..{rows - 1} equal to the oracle: {same}; CPU AVX2 product of {rows} rows "
            f"{cpu_s * 1e3:.2f} ms")
        if not same:
            log("PARITY FAILURE")
            sys.exit(1)
        results.append(dict(M=M, us=round(us, 3), tops=round(ops / us / 1e6, 2),
                            cpu_ms_256_rows=round(cpu_s * 1e3, 3), equal_to_oracle=same))
    big = results[-1]
    print(json.dumps({
        "metric": "int8 c_attn GEMM with requantize epilogue on 1 MI355X (K 768, N 2304)",
        "value": big["tops"], "unit": "TOPS", "n_gpus": 1, "steps": 50, "warmup": 10,
        "ms_per_step": round(big["us"] / 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "c_attn GEMM, A [M, 768] x W [2304, 768] i8, bias, rescale shift 42",
                   "shapes": results},
        "roofline": {"bound": "mfma", "kernel": "k_gemm<Act>", "achieved": big["tops"],
                     "peak": INT8_PEAK_TOPS, "unit": "TFLOP/s",
                     "frac": round(big["tops"] / INT8_PEAK_TOPS, 4), "traffic": None},
        "cpu_baseline": {"value": round(2 * 256 * N * K / (results[0]["cpu_ms_256_rows"] * 1e9), 4),
                         "unit": "TOPS", "cores": 1, "kind": "port",
                         "sample": "the oracle's AVX2 product of 256 rows (one thread)"},
    }), flush=True)


VENDOR_SHAPES = (  # (name, M, K, N): the GPT-2-small fold's products, and one decode pass's c_attn
    ("c_attn", 16384, 768, 2304), ("c_proj", 16384, 768, 768), ("c_fc", 16384, 768, 3072),
    ("mlp.c_proj", 16384, 3072, 768), ("lm_head (N padded to 50,304)", 2048, 768, 50304),
    ("c_attn, decode pass", 256, 768, 2304))


def run_gemm_vendor(args):
    """The fold's GEMM shapes on this build's k_gemm (i8 x i8 -> i32, bias, per-channel rescale,
    clamp to +-127: the Act epilogue, i8 outputs) and on the vendor library's int8 product
    (hipBLASLt through torch._int_mm: i8 x i8 -> i32, no epilogue, 4 B written per output).
    Both on the same operands, timed with hipEvents over 20 launches (the best of 3 runs); rows
    0..63 of each are checked against the oracle's exact product. torch is only the comparator
    here: the fold path never calls it."""
    import torch
    from oracle import oracle as O
    from taco_amd import hip
    dev = hip.HipDevice.open(0)
    rng = np.random.default_rng(0xBEEF)
    rows, total_ops, ours_us, lib_us = [], 0, 0.0, 0.0
    for name, M, K, N in VENDOR_SHAPES:
        w = rng.integers(-127, 128, (N, K)).astype(np.int8)
        a = rng.integers(-127, 128, (M, K)).astype(np.int8)
        bias = rng.integers(-(1 << 16), (1 << 16) + 1, N).astype(np.int32)
        mult = rng.integers(1 << 30, 1 << 31, N).astype(np.int64).astype(np.int32)
        shift = 42
        mp, np_, kp = hip.gemm_layout(M, N, K)
        bufs = [_dev_buf(hip, dev, x) for x in (hip.gemm_pack(w, np_, kp), hip.gemm_pack(a, mp, kp), bias, mult)]
        out = np.zeros((M, N), np.int8)
        dout = _dev_buf(hip, dev, out)
        ns = C.c_uint64()
        hip._check(hip.lib().hs_op_gemm_requant_gpu_ns(dev.h, bufs[0], bufs[1], bufs[2], bufs[3], shift,
                                                         M, N, K, dout, 5, C.byref(ns)))
        best = float("inf")
        for _ in range(3):
            hip._check(hip.lib().hs_op_gemm_requant_gpu_ns(dev.h, bufs[0], bufs[1], bufs[2], bufs[3], shift,
                                                             M, N, K, dout, 20, C.byref(ns)))
            best = min(best, ns.value / 20 / 1e3)
        hip._check(hip.lib().hs_device_download(dev.h, out.ctypes.data_as(C.c_void_p), dout, out.nbytes))
        for p in bufs + [dout]:
            hip.lib().hs_device_free(dev.h, p)
        ours_ok = bool(np.array_equal(out[:64], O.linear_act_ref(w, a[:64], bias, mult, shift)))
        ta = torch.from_numpy(a).cuda()
        tb = torch.from_numpy(w).cuda().t()  # [K, N], column-major: the NT product
        for _ in range(5):
            tc = torch._int_mm(ta, tb)
        torch.cuda.synchronize()
        lbest = float("inf")
        for _ in range(3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(20):
                tc = torch._int_mm(ta, tb)
            e1.record()
            torch.cuda.synchronize()
            lbest = min(lbest, e0.elapsed_time(e1) * 1e3 / 20)
        lib_ok = bool(np.array_equal(tc[:64].cpu().numpy().astype(np.int64), O.matmul_i8(w, a[:64])))
        del ta, tb, tc
        ops = 2 * M * N * K
        total_ops += ops
        ours_us += best
        lib_us += lbest
        log(f"{name:30s} M {M:5d} K {K:4d} N {N:5d}: k_gemm {best:8.2f} us {ops / best / 1e6:7.1f} TOPS "
            f"(rows 0..63 exact: {ours_ok}); hipBLASLt {lbest:8.2f} us {ops / lbest / 1e6:7.1f} TOPS "
            f"(rows 0..63 exact: {lib_ok}); {lbest / best:.2f}x")
        if not (ours_ok and lib_ok):
            log("PARITY FAILURE")
            sys.exit(1)
        rows.append(dict(name=name, M=M, K=K, N=N, k_gemm_us=round(best, 3),
                         k_gemm_tops=round(ops / best / 1e6, 1), hipblaslt_us=round(lbest, 3),
                         hipblaslt_tops=round(ops / lbest / 1e6, 1), speedup=round(lbest / best, 3)))
    agg = total_ops / ours_us / 1e6
    print(json.dumps({
        "metric": "int8 GEMM of the fold's shapes on 1 MI355X: fused requantize kernel vs hipBLASLt",
        "value": round(agg, 1), "unit": "TOPS", "n_gpus": 1, "steps": 20, "warmup": 5,
        "ms_per_step": round(ours_us / 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "the GPT-2-small fold's GEMM shapes (M 16,384; the LM head at 2,048 "
                               "rows) and the decode c_attn (M 256), Act epilogue vs torch._int_mm",
                   "shapes": rows},
        "vendor": {"library": "hipBLASLt through torch._int_mm (i32 outputs, no epilogue)",
                   "tops": round(total_ops / lib_us / 1e6, 1),
                   "time_ratio": round(lib_us / ours_us, 3)},
        "roofline": {"bound": "mfma", "kernel": "k_gemm<Act>", "achieved": round(agg, 1),
                     "peak": INT8_PEAK_TOPS, "unit": "TFLOP/s", "frac": round(agg / INT8_PEAK_TOPS, 4),
                     "traffic": None},
        "cpu_baseline": None,
    }), flush=True)


ISSUE_OPS = (("v_add_u32", 8, None), ("v_mad_i64_i32", 8, None), ("v_fma_f64", 8, None),
             ("v_mfma_i32_16x16x64_i8", 8, 16), ("v_mfma_i32_32x32x32_i8", 4, 32),
             ("v_ashrrev_i64", 8, None), ("v_mul_hi_i32", 8, None))
# ops 7 and 8: MFMA chains on waves 0-3 of an 8-wave workgroup, VALU chains (3x the rounds) on
# waves 4-7
MIXED_OPS = ((7, "mfma + v_add_u32"), (8, "mfma + v_mad_i64_i32"))


def run_issue(args):
    """Issue rates (hs_probe_issue): clocks per instruction per SIMD at the nominal 2.4 GHz for
    three VALU forms and the two int8 MFMA forms, at 1, 2 and 4 waves per SIMD. An MFMA form's
    peak is 16 (16 x 16 x 64) or 32 (32 x 32 x 32) clocks per instruction: 5.0 POPS over 1,024
    SIMDs at 2.4 GHz is 2,035 int8 ops per clock and SIMD."""
    from taco_amd import hip
    dev = hip.HipDevice.open(0)
    iters = 4096
    rows = []
    for op, (name, per_round, peak_clk) in enumerate(ISSUE_OPS):
        for wps in (1, 2, 4):
            ns = min(hip.probe_issue(dev, op, wps, iters) for _ in range(3))
            inst = wps * iters * per_round  # per SIMD
            clk = ns * 1e-9 * 2.4e9 / inst
            row = {"op": name, "waves_per_simd": wps, "ns": ns, "clocks_per_instruction": round(clk, 2)}
            if peak_clk:
                row["frac_of_peak_rate"] = round(peak_clk / clk, 3)
            rows.append(row)
            log(f"{name:24s} {wps} waves/SIMD: {clk:6.2f} clocks per instruction"
                + (f" ({peak_clk / clk:.3f} of the peak rate)" if peak_clk else ""))
    # Mixed: alone, the MFMA waves take T_m (op 3 at one wave per SIMD) and the VALU waves T_v
    # (the VALU op at one wave per SIMD, 3x the rounds); the mixed time against max and sum
    # tells whether the two kinds issue side by side on a SIMD.
    mixed = []
    for op, name in MIXED_OPS:
        ns = min(hip.probe_issue(dev, op, 2, iters) for _ in range(3))
        t_m = min(hip.probe_issue(dev, 3, 1, iters) for _ in range(3))
        t_v = min(hip.probe_issue(dev, 0 if op == 7 else 1, 1, 3 * iters) for _ in range(3))
        mixed.append({"ops": name, "ns": ns, "mfma_alone_ns": t_m, "valu_alone_ns": t_v,
                      "overlap": round((t_m + t_v - ns) / min(t_m, t_v), 3)})
        log(f"{name}: {ns} ns; alone {t_m} and {t_v} ns; overlap {mixed[-1]['overlap']} "
            "(1: fully side by side, 0: one after the other)")
    big = [r for r in rows if r["op"] == "v_mfma_i32_16x16x64_i8" and r["waves_per_simd"] == 2][0]
    line = {"metric": "int8 MFMA issue rate on 1 MI355X (v_mfma_i32_16x16x64_i8, 2 waves per SIMD)",
            "value": big["frac_of_peak_rate"], "unit": "fraction of the peak rate", "n_gpus": 1,
            "steps": 3, "warmup": 1, "ms_per_step": round(big["ns"] / 1e6, 4), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic",
            "config": {"workload": "issue-rate probe: 4,096 rounds per wave, 256 x waves workgroups",
                       "rows": rows, "mixed": mixed},
            "roofline": None, "cpu_baseline": None}
    print(json.dumps(line), flush=True)


def run_attend(args):
    """Decode attention, one query row per stream: 64 streams x 12 heads x 64 over caches of
    ctx positions, rotating over cache sets that together exceed the 256 MB Infinity Cache."""
    from oracle import oracle as O
    from taco_amd import hip
    dev = hip.HipDevice.open(0)
    rng = np.random.default_rng(0xC3)
    B, H, hd = 64, 12, 64
    table = np.array([round(2 ** 30 * np.exp(-i / 256)) for i in range(8192)], np.int32)
    score_m, score_s, out_m, out_s = 1_400_000_000, 34, 1_300_000_000, 53
    dtab = _dev_buf(hip, dev, table)
    rows = []
    if args.calib_copy_mib:
        calibration_copy(hip, dev, args.calib_copy_mib)
    for ctx, sets in ATTEND_CONTEXTS:
        assert sets == max(3, (768 << 20) // (2 * B * H * ctx * hd))  # >= 768 MB of caches
        q = rng.integers(-127, 128, (B, H, hd)).astype(np.int8)
        ctxs = np.full(B, ctx, np.uint32)
        dq, dctx = _dev_buf(hip, dev, q), _dev_buf(hip, dev, ctxs)
        caches = []
        for s in range(sets):
            kc = rng.integers(-127, 128, (B, H, ctx, hd)).astype(np.int8)
            vc = rng.integers(-127, 128, (B, H, ctx, hd)).astype(np.int8)
            caches.append((kc, vc, _dev_buf(hip, dev, kc), _dev_buf(hip, dev, vc)))
        out = np.zeros((B, H * hd), np.int8)
        dout = _dev_buf(hip, dev, out)
        ns = C.c_uint64()
        dks = (C.c_void_p * sets)(*[c[2] for c in caches])
        dvs = (C.c_void_p * sets)(*[c[3] for c in caches])
        for r in range(2):  # one launch per set in turn, back to back: every launch reads cold
            hip._check(hip.lib().hs_op_attend_decode_sets_gpu_ns(  # caches; round 0 warms up
                dev.h, dq, dks, dvs, sets, dctx, B, H, hd, ctx, score_m, score_s, out_m, out_s,
                dtab, len(table), 30, dout, C.byref(ns)))
        total, reps = ns.value, sets
        hip._check(hip.lib().hs_device_download(dev.h, out.ctypes.data_as(C.c_void_p), dout,
                                                out.nbytes))
        kc, vc = caches[sets - 1][:2]  # the last launch wrote out
        ts = time.perf_counter()
        want = O.attend_decode_ref(q, kc, vc, ctxs, score_m, score_s, out_m, out_s, table, 30)
        cpu_s = time.perf_counter() - ts
        same = bool(np.array_equal(out, want))
        us = total / reps / 1e3
        nbytes = 2 * B * H * ctx * hd + 2 * B * H * hd
        gbs = nbytes / us / 1e3
        log(f"attend ctx {ctx}: {us:.2f} us per launch over {sets} cache sets, {gbs:.0f} GB/s, "
            f"equal to the oracle: {same}; oracle {cpu_s * 1e3:.1f} ms")
        if not same:
            log("PARITY FAILURE")
            sys.exit(1)
        rows.append(dict(ctx=ctx, us=round(us, 3), gbs=round(gbs, 1), bytes=nbytes,
                         cache_sets=sets, cpu_ms=round(cpu_s * 1e3, 2), equal_to_oracle=same))
        for _, _, dk, dv in caches:
            hip.lib().hs_device_free(dev.h, dk)
            hip.lib().hs_device_free(dev.h, dv)
        for p in (dq, dctx, dout):
            hip.lib().hs_device_free(dev.h, p)
    hip.lib().hs_device_free(dev.h, dtab)
    # the stream-read probe (read_gpu_ns, ops.rs:328-335): 2 GiB, well beyond the Infinity Cache
    stream = hip.read_bw(dev, 2 << 30, 10) / 1e9
    log(f"stream read: {stream:.0f} GB/s")
    big = rows[-1]
    print(json.dumps({
        "metric": "integer decode attention over an HBM KV cache on 1 MI355X (64 x 12 x 64)",
        "value": big["gbs"], "unit": "GB/s", "n_gpus": 1, "steps": rows[-1]["cache_sets"],
        "warmup": rows[-1]["cache_sets"], "ms_per_step": round(big["us"] / 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "decode attention, 64 streams x 12 heads x 64, ctx sweep",
                   "contexts": rows},
        "roofline": {"bound": "hbm", "kernel": "k_attend_decode64 (1,024 keys)", "achieved": big["gbs"],
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(big["gbs"] / HBM_PEAK_GBS, 4),
                     "stream_read_gbs": round(stream, 1),
                     "frac_of_stream_read": round(big["gbs"] / stream, 4),
                     "traffic": committed_attend_traffic(big["ctx"]),
                     "traffic_unit": "HBM bytes per launch at the largest context (FETCH_SIZE + "
                                     "WRITE_SIZE, calibrated; profiles/attend_decode_traffic.json)"},
        "cpu_baseline": {"value": round(big["bytes"] / (big["cpu_ms"] * 1e6), 3), "unit": "GB/s",
                         "cores": 1, "kind": "port",
                         "sample": "the oracle's scalar decode attention of one cache set"},
    }), flush=True)


def main_traffic(argv):
    """python bench.py --traffic-summary FETCH.csv WRITE.csv CALIB_MIB WORKLOAD: the summary of
    two rocprofv3 counter runs of `bench.py --workload WORKLOAD --calib-copy-mib CALIB_MIB`."""
    from taco_amd import synth
    fetch_csv, write_csv, calib, workload = argv
    if workload == "attend-decode":
        cmd = ("rocprofv3 --pmc FETCH_SIZE (then WRITE_SIZE) --output-format csv -- python3 bench.py "
               f"--workload attend-decode --steps 1 --warmup 0 --no-cpu --calib-copy-mib {calib}")
        print(json.dumps(attend_traffic_summary(fetch_csv, write_csv, int(calib), cmd), indent=1))
        return
    dims_name, W, n, _ = FOLDS[workload]
    tokens_sha = synth.sha256_tokens(synth.zipf_tokens(W * n))
    cmd = (f"rocprofv3 --pmc FETCH_SIZE (then WRITE_SIZE) --output-format csv -- python3 bench.py "
           f"--workload {workload} --steps 1 --warmup 0 --no-cpu --batches 1 --calib-copy-mib {calib}")
    print(json.dumps(traffic_summary(fetch_csv, write_csv, int(calib), tokens_sha, cmd), indent=1))


def main_mfma(argv):
    """python bench.py --mfma-summary COUNTERS.csv WORKLOAD: the MFMA summary of one rocprofv3
    --pmc run of `bench.py --workload WORKLOAD --steps 1 --warmup 0 --no-cpu --sustain-s 0`."""
    from taco_amd import synth
    csv_path, workload = argv
    dims_name, W, n, _ = FOLDS[workload]
    tokens_sha = synth.sha256_tokens(synth.zipf_tokens(W * n))
    cmd = ("rocprofv3 --pmc SQ_INSTS_VALU_MFMA_MOPS_I8 SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE "
           "SQ_BUSY_CYCLES --output-format csv -- python3 bench.py --workload " + workload +
           " --steps 1 --warmup 0 --no-cpu --no-unfold --sustain-s 0 --batches 1")
    print(json.dumps(mfma_summary(csv_path, tokens_sha, cmd), indent=1))


def main_sq(argv):
    """python bench.py --sq-summary PASS1.csv PASS2.csv WORKLOAD: the instruction-mix summary of
    the two rocprofv3 --pmc runs of SQ_PASSES over `bench.py --workload WORKLOAD --steps 1
    --warmup 0 --no-cpu --no-unfold --sustain-s 0`."""
    from taco_amd import synth
    a_csv, b_csv, workload = argv
    dims_name, W, n, _ = FOLDS[workload]
    tokens_sha = synth.sha256_tokens(synth.zipf_tokens(W * n))
    cmd = " ; ".join("rocprofv3 --pmc " + " ".join(p) + " --output-format csv -- python3 bench.py --workload "
                     + workload + " --steps 1 --warmup 0 --no-cpu --no-unfold --sustain-s 0 --batches 1"
                     for p in SQ_PASSES)
    print(json.dumps(sq_summary([a_csv, b_csv], tokens_sha, cmd), indent=1))


def main():
    if len(sys.argv) > 1 and sys.argv[1] == "--sq-summary":
        return main_sq(sys.argv[2:])
    if len(sys.argv) > 1 and sys.argv[1] == "--traffic-summary":
        return main_traffic(sys.argv[2:])
    if len(sys.argv) > 1 and sys.argv[1] == "--mfma-summary":
        return main_mfma(sys.argv[2:])
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=80)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--workload", default="fold-gpt2-small",
                    choices=sorted(FOLDS) + ["gemm-qkv", "gemm-vendor", "attend-decode", "issue-rates"])
    ap.add_argument("--windows", type=int, default=0)
    ap.add_argument("--window-tokens", type=int, default=0)
    ap.add_argument("--cpu-windows", type=int, default=0,
                    help="windows in the CPU-baseline sample (0: the workload's default)")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--sustain-s", type=float, default=3.0,
                    help="seconds of fold steps after the timed ones for the sustained figure")
    ap.add_argument("--no-unfold", action="store_true")
    ap.add_argument("--batches", type=int, default=4,
                    help="fold batches in flight, each on its own host thread and stream")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="first copy this many MiB device to device (the known-size copy that "
                         "scales FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for {args.gpus}): the fold shards by windows "
              "with no exchange between GPUs, and this build measures the one-GPU share",
              file=sys.stderr)
        sys.exit(2)
    if args.workload in FOLDS:
        run_fold(args)
    elif args.workload == "gemm-qkv":
        run_gemm(args)
    elif args.workload == "gemm-vendor":
        run_gemm_vendor(args)
    elif args.workload == "issue-rates":
        run_issue(args)
    else:
        run_attend(args)


if __name__ == "__main__":
    main()
