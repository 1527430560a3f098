#!/usr/bin/env python3
"""Fold throughput of the HardShell hot path on one MI355X.

Workload (the north-star configuration): a GPT-2-small-shape integer model in .hsm layout
(12 layers, d_model 768, 12 heads x 64, d_ff 3072, vocab 50,257, n_ctx 1,024) with seeded
uniform int8 weights, folding a 16,384-token Zipf(1.1) stream as 64 independent 256-token
windows (blocks of 1,024 bytes of fixed-width 4-byte tokens) batched on one GPU. One step is
one whole fold: the integer forward pass of all 16,384 rows, the logits -> CDF coder op on the
GPU, the host range coder, the block payloads and the .taco container.

Prints one JSON line. `value` is fold tokens per second with the token stream and the model
already resident (model upload and token staging are outside the timed region; per step the
host sends 8 B and receives 24 B per token). `roofline` is the int8 GEMM kernels against the
MI355X dense int8 MFMA peak, from hipEvents around every launch in the timed steps.
`cpu_baseline` is the oracle's C++ restatement of the reference CPU fast path (AVX2 products,
prefill chunk 32, one window per thread) timed on a sample of the same windows in the same run;
its payloads must equal the GPU's.
"""

import argparse
import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA, 5.0 POPS
HBM_PEAK_GBS = 8000.0


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--windows", type=int, default=64)
    ap.add_argument("--window-tokens", type=int, default=256)
    ap.add_argument("--cpu-windows", type=int, default=0,
                    help="windows in the CPU-baseline sample (0: one per thread)")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="first copy this many MiB device to device (the known-size copy that "
                         "scales FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for {args.gpus}): the fold shards by windows "
              "with no exchange between GPUs, and this build measures the one-GPU share",
              file=sys.stderr)
        sys.exit(2)

    from taco_amd import fold, hip, synth

    t0 = time.time()
    dims = synth.GPT2_SMALL
    model_bytes = synth.build_model(dims)
    W, n = args.windows, args.window_tokens
    tokens = synth.zipf_tokens(W * n)
    blocks = [tokens[w * n:(w + 1) * n] for w in range(W)]
    original = fold.token_bytes(tokens)
    block_size = 4 * n
    log(f"workload built in {time.time() - t0:.1f}s: model {len(model_bytes)} B "
        f"sha256 {hashlib.sha256(model_bytes).hexdigest()[:16]}, tokens sha256 "
        f"{synth.sha256_tokens(tokens)[:16]}")

    dev = hip.HipDevice.open(0)
    if args.calib_copy_mib:
        import ctypes as C
        nb = args.calib_copy_mib << 20
        src, dst = C.c_void_p(), C.c_void_p()
        hip._check(hip.lib().hs_device_alloc(dev.h, nb, C.byref(src)))
        hip._check(hip.lib().hs_device_alloc(dev.h, nb, C.byref(dst)))
        hip._check(hip.lib().hs_device_copy(dev.h, dst, src, nb))
        hip.lib().hs_device_free(dev.h, src)
        hip.lib().hs_device_free(dev.h, dst)
        log(f"calibration copy: {args.calib_copy_mib} MiB device to device")
    model = hip.HipModel.load(dev, model_bytes)
    batch = hip.HipBatch(model, W, W * n)
    log(f"device {dev.name()}, model {model.weight_bytes() / 1e6:.1f} MB, batch "
        f"{batch.gpu_bytes() / 1e9:.2f} GB")

    phase = {"fold": 0.0, "container": 0.0}

    def step():
        t0 = time.perf_counter()
        payloads = fold.fold_blocks(batch, blocks, 0)  # every row runs (no early stop)
        t1 = time.perf_counter()
        cont = fold.container(model.hash(), original, block_size, 0, payloads)
        phase["fold"] += t1 - t0
        phase["container"] += time.perf_counter() - t1
        return payloads, cont

    for i in range(args.warmup):
        ts = time.time()
        payloads, cont = step()
        log(f"warmup {i}: {time.time() - ts:.3f}s, container {len(cont)} B")
    hip._check(hip.lib().hs_batch_set_profiling(batch.h, 1))
    hip.lib().hs_batch_profile(batch.h, None, None, None, None, 0, 1)
    phase.update(fold=0.0, container=0.0)
    ts = time.perf_counter()
    for i in range(args.steps):
        payloads, cont = step()
    elapsed = time.perf_counter() - ts
    hip._check(hip.lib().hs_batch_set_profiling(batch.h, 0))
    import ctypes as C
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
    gemm_ns = sum(v["ns"] for kk, v in prof.items() if kk.startswith("gemm"))
    gemm_ops = sum(v["ops"] for kk, v in prof.items() if kk.startswith("gemm"))
    gemm_launches = sum(v["launches"] for kk, v in prof.items() if kk.startswith("gemm"))
    achieved = gemm_ops / gemm_ns / 1e3 if gemm_ns else 0.0  # ops/ns -> TOPS
    tokens_per_step = W * n
    value = tokens_per_step * args.steps / elapsed
    cont_sha = hashlib.sha256(cont).hexdigest()
    coded = sum(1 for p in payloads if p is not None and len(p) < block_size)
    log(f"timed: {args.steps} steps in {elapsed:.3f}s -> {value:.0f} tokens/s; container "
        f"{len(cont)} B sha256 {cont_sha[:16]}, {coded}/{W} blocks coded")
    gpu_ms = sum(v["ns"] for v in prof.values()) / 1e6 / args.steps
    log(f"  per step: fold call {1e3 * phase['fold'] / args.steps:.3f} ms (kernels {gpu_ms:.3f} ms), "
        f"container {1e3 * phase['container'] / args.steps:.3f} ms")
    for kk, v in sorted(prof.items(), key=lambda x: -x[1]["ns"]):
        log(f"  {kk:12s} {v['ns'] / 1e6 / args.steps:8.3f} ms/step  {v['launches'] // args.steps:5d} "
            f"launches/step" + (f"  {v['ops'] / v['ns'] / 1e3:7.1f} TOPS" if v["ops"] and v["ns"] else ""))

    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O
        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
        cw = args.cpu_windows or 2 * threads
        cw = min(cw, W)
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
        cpu = {"value": round(cw * n / cpu_s, 2), "unit": "tokens/s", "cores": threads,
               "kind": "port",
               "sample": f"the first {cw} of the {W} windows ({cw * n} tokens), two windows per "
                         f"thread, AVX2 restatement of the reference CPU fast path, chunk 32",
               "payloads_equal_gpu": same}

    out = {
        "metric": "fold tokens/sec on 1 MI355X (GPT-2 124M int8, bit-exact); int8 MFMA % of peak",
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
        "config": {"workload": f"gpt2-small-shape fold: {W} windows x {n} Zipf(1.1) tokens",
                   "layers": dims.n_layer, "d_model": dims.d_model, "heads": dims.n_head,
                   "d_ff": dims.d_ff, "vocab": dims.vocab, "n_ctx": dims.n_ctx,
                   "tokens_per_step": tokens_per_step, "container_sha256": cont_sha,
                   "tokens_sha256": synth.sha256_tokens(tokens)},
        "roofline": {"bound": "mfma", "kernel": "k_gemm (all int8 GEMMs of the pass)",
                     "achieved": round(achieved, 2), "peak": INT8_PEAK_TOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / INT8_PEAK_TOPS, 4),
                     "traffic": None, "launches": gemm_launches,
                     "ops_per_launch": gemm_ops // max(1, gemm_launches),
                     "avg_launch_us": round(gemm_ns / max(1, gemm_launches) / 1e3, 2)},
        "ops_ms_per_step": {kk: round(v["ns"] / 1e6 / args.steps, 3) for kk, v in prof.items()},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
