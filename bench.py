"""Benchmark: sampled rows/s of the GPU sampler on one MI355X.

A step is one pick over the whole batch of the workload (default: peaked_b256, the
batch-256 full-sampler workload): repeat penalty, temperature, top-k, softmax, top-p,
min-p and the seeded draw for every row, logits already resident in HBM.  The timed
region is `--steps` back-to-back picks between two HIP events on the sampler's stream,
with a device synchronisation on both sides, after --settle-s seconds of untimed picks
(the GPU leaves the idle clocks it sits at after input generation; a short warm-up of a
few picks does not bring it up) and `--warmup` untimed steps.  Generator states and
histories evolve from step to step, as in decoding.  The CPU baseline runs after the
GPU timing.

MI355X keeps up to 256 MiB in its last-level cache (Infinity Cache), which would hold one
batch-256 logits array whole; the picks therefore rotate over enough copies of the
input (--buffers, default: more than 512 MiB in total) that each pick reads from HBM.
--buffers 1 measures the warm-cache case.

Also reported on the same JSON line:
  roofline      for the pick's dominant kernel (the row kernel k_row, the whole pick, or
                the streaming kernel k_part): algorithmic bytes per launch (4V logits + 4H
                history + 4 id + 16 RNG per row) over its average duration, against 8 TB/s
                HBM.  The row kernel is one launch a step: its average duration is the timed
                region's (HIP events on the batch's stream over the back-to-back launches);
                `kernel_ms_isolated` is each of --kernel-steps further launches timed alone
                (an event before it, one after it), which adds a start from an idle queue.
                The streaming kernel k_part is timed alone that way, with an event between
                the pick's two kernels.  `pick_frac` is the same bytes over the whole pick;
                `traffic` is the HBM bytes per pick that hardware counters
                measured for the same workload and kernels (profiles/traffic.json, written
                from rocprofv3 FETCH_SIZE and WRITE_SIZE runs scaled by the same counters
                on a copy of known size; null when no such measurement is committed)
  read_ceiling  when the pick is the row kernel at one row per CU: the same rows read by
                a kernel with the row kernel's launch shape, chunks and loads that only
                adds them up (qs_time_row_reads), its time and rate, and the pick's time
                over it (the part of the pick the sampling itself costs)
  cpu_baseline  the reference's own sample.c (oracle/_ref, when built) or the CPU
                restatement over a bounded sample of the same rows, on the host's cores
                (at most 16 threads: a one-GPU share of the box) and on one core, with the
                host's CPU model
  parity        the first step's ids and per-row intermediates against the CPU
                restatement on every row: id mismatches, draws within 1e-6 of a CDF
                boundary, mismatches not explained by one, normalisers outside the GPU's
                (proven) value or interval, kept-prefix mismatches
Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--rows B]
                       [--mode M]
       python bench.py --calibrate-copy [--copy-mib N]   (copies of N MiB, for the counters)
       python bench.py --router [--router-tokens T]      (the MoE router's expert choice:
                                                           T tokens x 128 experts, top 8)
       python bench.py --head [--head-rows B]            (the output layer and the pick:
                                                           B x 2048 hidden states, a
                                                           151,936 x 2048 bf16 matrix)
       python bench.py --sample-h [--workload full_b1]   (sample.h's pick end to end:
                                                           host logits in, id out)
       python bench.py --head-exact [--head-exact-rows B] (the output layer at the
                                                           reference's arithmetic, B <= 8
                                                           rows, a Q6_K 151,936 x 2048
                                                           matrix, and the pick)
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "sampled rows/s at B={B}, V={V} fp32; achieved HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0
CACHE_DEFEAT_BYTES = 512 << 20       # twice the MI355X last-level cache


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--workload", default=None)
    ap.add_argument("--rows", type=int, default=0,
                    help="the workload's settings at this batch size (0: its own)")
    ap.add_argument("--settle-s", type=float, default=0.25,
                    help="untimed picks for this long before the warm-up steps: the GPU "
                         "leaves the idle clocks of input generation (0: none)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="approximate CPU work for the baseline sample")
    ap.add_argument("--cpu-threads", type=int, default=0, help="0: all host cores (<= 16)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--buffers", type=int, default=0,
                    help="input copies the timed picks rotate over (0: enough to exceed "
                         "twice the last-level cache)")
    ap.add_argument("--mode", choices=["auto", "split", "stream", "row"], default="auto",
                    help="which kernels a pick uses (qs_batch_set_mode)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run plain device copies of --copy-mib MiB (counter calibration)")
    ap.add_argument("--copy-mib", type=int, default=512)
    ap.add_argument("--copy-kind", choices=["plain", "buffer", "lds", "dword"],
                    default="plain",
                    help="the calibration copy's load: plain 16-byte global loads, "
                         "nontemporal raw buffer loads (the row kernel's), those loads into "
                         "LDS (the streaming part kernel's), or plain 4-byte loads")
    ap.add_argument("--router", action="store_true",
                    help="only time qs_router_topk (128 experts, 8 used, renormalised)")
    ap.add_argument("--router-tokens", type=int, default=4096)
    ap.add_argument("--head", action="store_true",
                    help="the output layer with the pick (fused) against the layer then a pick")
    ap.add_argument("--head-rows", type=int, default=256)
    ap.add_argument("--head-exact", action="store_true",
                    help="the output layer at the reference's arithmetic and the pick")
    ap.add_argument("--head-exact-rows", type=int, default=1)
    ap.add_argument("--sample-h", action="store_true",
                    help="end-to-end latency of sample.h's quasar_sampler_pick (host logits "
                         "in, id out) on the workload's settings (default full_b1)")
    ap.add_argument("--kernel-steps", type=int, default=100,
                    help="picks timed kernel by kernel for the roofline")
    return ap.parse_args()


KERNELS = {"split": "k_scan + k_expsum + k_finalize", "stream": "k_part + k_decide",
           "row": "k_row"}
MODE_NAMES = {1: "split", 2: "stream", 3: "row"}


def calibrate_copy(args):
    """Plain copies of known size: their FETCH_SIZE / WRITE_SIZE per dispatch calibrate the
    counters that measure a pick's HBM traffic."""
    import quasar_amd as qa
    n = args.copy_mib << 20
    src, dst = qa.DeviceBuffer(n), qa.DeviceBuffer(n)
    kind = {"plain": 0, "buffer": 1, "lds": 2, "dword": 3}[args.copy_kind]
    qa.copy_device(dst, src, n, 4, kind)
    print(json.dumps({"calibrate_copy": {"bytes_read": n, "bytes_written": n, "copies": 4,
                                         "load": args.copy_kind}}), flush=True)


def committed_traffic(workload, mode):
    """HBM bytes per pick measured by counters for this workload and kernel, if committed."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f).get(f"{workload}/{mode}")
    except (OSError, ValueError):
        return None
    return t


def host_cpu():
    """(CPUs this process may run on, CPUs of the host, the CPU model name)."""
    try:
        usable = len(os.sched_getaffinity(0))
    except OSError:
        usable = os.cpu_count() or 1
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return usable, os.cpu_count() or usable, model


def cpu_baseline(w, logits_host, hist, seeds, gpu_ids, gpu_diag, args):
    """Time the reference sampler (or the restatement) on the host: one untimed warm-up
    pass, then at least 5 timed passes (until about args.cpu_seconds of work), on as many
    threads as the process may use (nproc) and on one; the rate is the median pass's.
    Check the GPU's first-step ids and intermediates against the restatement on every
    row."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from pyoracle import Oracle, Params, RefSampler, parity_report
    if RefSampler.available():
        impl, kind = RefSampler(), "reference"
    else:
        impl, kind = Oracle(), "port"
    p = Params(*[w.temperature, w.top_p, w.min_p, w.repeat_penalty], w.top_k, w.repeat_last_n)
    usable, host_cpus, model = host_cpu()
    threads = args.cpu_threads or usable
    B, V = logits_host.shape

    def timed(n_threads, rows, budget):
        """(median rows/s over the timed passes, rows per pass, passes, seconds)"""
        impl.pick_rows(p, logits_host, rows, V, hist, seeds, n_threads)    # warm-up
        rates, secs = [], 0.0
        while len(rates) < 5 or (secs < budget and len(rates) < 200):
            _, s_ = impl.pick_rows(p, logits_host, rows, V, hist, seeds, n_threads)
            rates.append(rows / s_)
            secs += s_
        return float(np.median(rates)), rows, len(rates), secs

    rate, _, reps, secs = timed(threads, B, args.cpu_seconds)
    # one core: passes of about a fifth of a quarter of the budget each
    one_rows = max(1, min(B, int(rate / threads * args.cpu_seconds / 20)))
    rate1, _, reps1, secs1 = timed(1, one_rows, args.cpu_seconds / 4)
    orc_ids, orc_diag, _ = Oracle().pick_rows_diag(p, logits_host, B, V, hist, seeds, threads)
    parity = parity_report(gpu_ids, gpu_diag, orc_ids, orc_diag)
    base = {"value": rate, "unit": "rows/s", "cores": threads, "kind": kind,
            "single_core": rate1, "host_cpus": host_cpus, "cpu_model": model,
            "sample": f"median of {reps} timed passes (after one warm-up pass) over all {B} "
                      f"rows of {w.name} ({secs:.1f} s of pick time) on {threads} POSIX "
                      f"threads (nproc {usable}), one sampler per row; single core: median "
                      f"of {reps1} passes over the first {one_rows} rows ({secs1:.1f} s)"}
    return base, parity


def router_bench(args):
    """The mixture-of-experts router's choice (qs_router_topk) on `--router-tokens`
    tokens of 128 router logits, 8 experts used, weights renormalised (a 128-expert,
    top-8 model's router per layer): tokens/s over back-to-back calls between HIP events,
    the output checked against the CPU restatement, which is also timed."""
    import quasar_amd as qa
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from pyoracle import Oracle
    T, E, U = args.router_tokens, 128, 8
    x = (np.random.default_rng(7).standard_normal((T, E)) * 3.0).astype(np.float32)
    buf = qa.DeviceBuffer.from_array(x)
    di, dw = qa.DeviceBuffer(4 * T * U), qa.DeviceBuffer(4 * T * U)
    qa.router_topk(buf, T, E, U, 1, di, dw)
    orc = Oracle()
    t0 = time.perf_counter()
    oi, ow = orc.router_topk(x, U, 1)
    cpu_s = time.perf_counter() - t0
    gi = di.download(np.int32, T * U).reshape(T, U)
    gw = dw.download(np.float32, T * U).reshape(T, U)
    mism = int(((gi != oi).any(axis=1) | (gw.view(np.uint32) != ow.view(np.uint32)).any(axis=1)).sum())
    qa.router_time(buf, T, E, U, 1, di, dw, args.warmup)
    ms = qa.router_time(buf, T, E, U, 1, di, dw, args.steps)
    us = ms * 1e3 / args.steps
    print(json.dumps({
        "metric": "MoE router choices/s (128 experts, top 8, renormalised)",
        "value": T / (us * 1e-6), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": us / 1e3, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "moe_router", "tokens": T, "experts": E, "used": U,
                   "norm_topk": True},
        "cpu_baseline": {"value": T / cpu_s, "unit": "tokens/s", "cores": 1, "kind": "port",
                         "sample": f"all {T} tokens once through the CPU restatement"},
        "parity": {"tokens_checked": T, "mismatches": mism}}), flush=True)
    for b_ in (buf, di, dw):
        b_.free()


def head_bench(args):
    """The output layer (LM head) and the pick: rows/s of qs_batch_pick_head (the layer with
    the sampler's first pass in its epilogue; the decision reads back only the tiles that
    hold candidates) against qs_batch_head_logits followed by qs_batch_pick, at B rows x
    n_embd 2048 x vocabulary 151,936 (a Qwen3 output layer), bf16 weights packed once, the
    peaked rows' sampler settings.  Checked before timing: the fused ids, generator states
    and histories equal the unfused pick's on the logits the call wrote, and sampled rows'
    logits lie within the fp32 summation bound of a float64 product on the host."""
    import quasar_amd as qa
    B, E, V = args.head_rows, 2048, 151936
    K, T, TOPP, MINP, RP, LASTN = 40, 0.8, 0.95, 0.05, 1.1, 256
    rng = np.random.default_rng(11)
    h32 = rng.standard_normal((B, E), dtype=np.float32) * np.float32(1.5)
    w32 = rng.standard_normal((V, E), dtype=np.float32) * np.float32(1.0 / np.sqrt(E))
    hb = (h32.view(np.uint32) >> 16).astype(np.uint16)           # bf16 by truncation
    wb = (w32.view(np.uint32) >> 16).astype(np.uint16)
    del w32
    hist = rng.integers(0, V, (B, LASTN)).astype(np.int32)
    seeds = qa.gen_row_seeds(17, 0, B)
    bats = [qa.Batch(B, V, LASTN) for _ in range(2)]
    dh, dwr = qa.DeviceBuffer.from_array(hb), qa.DeviceBuffer.from_array(wb)
    dw = qa.DeviceBuffer(qa.head_packed_bytes(E, V))
    bats[0].head_pack(dwr.ptr, E, V, dw.ptr)
    bats[0].synchronize()
    dwr.free()
    dl, dl2 = qa.DeviceBuffer(4 * B * V), qa.DeviceBuffer(4 * B * V)
    for bt in bats:
        bt.config(0, B, T, TOPP, K, MINP, RP, LASTN, seeds=seeds)
        bt.set_history(0, hist)
    # parity: one fused pick against the unfused pick on the logits it wrote
    ids_f = bats[0].pick_head(dh.ptr, dw.ptr, E, B, V, dl.ptr)
    logits = dl.download(np.float32, B * V).reshape(B, V)
    dl2.upload(logits)
    ids_p = bats[1].pick(dl2.ptr, V, B, V)
    mism = int((ids_f != ids_p).sum())
    mism += sum(int(bats[0].get_state(r)[0] != bats[1].get_state(r)[0]) for r in range(B))
    hf = (hb.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    wf = (wb.astype(np.uint32) << 16).view(np.float32)
    chk = list(range(0, B, max(1, B // 8)))
    bound_ok = True
    for c0 in range(0, V, 16384):                     # float64 products in column blocks
        wc = wf[c0:c0 + 16384].astype(np.float64)
        exact = wc @ hf[chk].T
        mag = np.abs(wc) @ np.abs(hf[chk]).T
        err = np.abs(logits[chk, c0:c0 + 16384].T - exact)
        bound_ok &= bool(np.all(err <= E * 2.0 ** -24 * mag + 1e-30))
    # the CPU path: the float32 product of one row and the restatement of sample.c
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from pyoracle import Oracle
    orc = Oracle()
    smp = orc.sampler()
    t0, n_cpu = time.perf_counter(), 0
    while n_cpu < 4 or time.perf_counter() - t0 < 3.0:
        row = wf @ hf[n_cpu % B].astype(np.float32)
        smp.config(T, TOPP, K, MINP, RP, LASTN, seed=1 + n_cpu)
        smp.pick(row)
        n_cpu += 1
    cpu_rate = n_cpu / (time.perf_counter() - t0)
    # timing: untimed settle, then each variant over --steps calls
    bats[0].time_head(dh.ptr, dw.ptr, E, B, V, dl.ptr, max(args.warmup, 20), 1)
    res = {}
    for name, mode in (("fused", 1), ("unfused", 0), ("layer_alone", 2)):
        bats[0].time_head(dh.ptr, dw.ptr, E, B, V, dl.ptr, 5, mode)
        res[name] = bats[0].time_head(dh.ptr, dw.ptr, E, B, V, dl.ptr, args.steps, mode) \
            * 1e3 / args.steps
    nt = (V + 127) // 128
    w_bytes = qa.head_packed_bytes(E, V)
    layer_bytes = w_bytes + 2 * B * E + 4 * B * V
    flops = 2.0 * B * V * E
    read_unfused = 4 * V                                 # the pick reads the whole row
    read_fused = (K + 2) * 128 * 4 + nt * 32             # K+2 tiles' logits + the records
    us_layer = res["layer_alone"]
    print(json.dumps({
        "metric": "output layer + pick rows/s (fused epilogue)",
        "value": B / (res["fused"] * 1e-6), "unit": "rows/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": res["fused"] / 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"lm_head_b{B}", "rows": B, "n_embd": E, "vocab": V,
                   "top_k": K, "temperature": T, "top_p": TOPP, "min_p": MINP,
                   "repeat_penalty": RP, "last_n": LASTN},
        "us": {k: round(v, 2) for k, v in res.items()},
        "roofline": {"kernel": "k_head (layer alone)", "bound": "hbm",
                     "achieved": layer_bytes / (us_layer * 1e-6) / 1e9, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": layer_bytes / (us_layer * 1e-6) / 1e9 / HBM_PEAK_GBS,
                     "mfma_tflops": flops / (us_layer * 1e-6) / 1e12, "mfma_peak": 2500.0,
                     "traffic": None},
        "logit_bytes_read_per_row": {"unfused": read_unfused, "fused": read_fused,
                                     "saved": read_unfused - read_fused},
        "cpu_baseline": {"value": cpu_rate, "unit": "rows/s", "cores": 1, "kind": "port",
                         "sample": f"{n_cpu} rows: numpy float32 product of the row with "
                                   "the matrix, then the restatement of sample.c"},
        "parity": {"rows": B, "fused_vs_unfused_mismatches": mism,
                   "logit_rows_within_fp32_bound": len(chk) if bound_ok else 0}}), flush=True)
    for b_ in (dh, dw, dl, dl2):
        b_.free()
    for bt in bats:
        bt.close()


def head_exact_bench(args):
    """The output layer at the reference's arithmetic and the pick: rows/s of
    qs_batch_pick_head_exact against qs_batch_head_exact_logits followed by qs_batch_pick,
    and the layer alone, at B (1..8) rows x n_embd 2048 x vocabulary 151,936 with the output
    matrix in Q6_K (the reference model's type), packed once.  Checked before timing: every
    logit of the fused call equals the CPU restatement of forward_cpu.c's gemv bit for bit,
    and the fused ids, generator states and histories equal the unfused pick's and the
    restatement's sampler on the same logits."""
    import quasar_amd as qa
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from pyoracle import Oracle
    B, E, V, WT = args.head_exact_rows, 2048, 151936, qa.WTYPE_Q6_K
    K, T, TOPP, MINP, RP, LASTN = 40, 0.8, 0.95, 0.05, 1.1, 256
    rng = np.random.default_rng(12)
    nb = E // 256
    wq = rng.integers(0, 256, (V, nb, 210), dtype=np.uint8)
    dsc = (rng.uniform(0.5, 1.5, (V, nb)) / 2048 / np.sqrt(E)).astype(np.float16)
    wq[:, :, 208:210] = dsc.view(np.uint8).reshape(V, nb, 2)
    wq = wq.reshape(V, nb * 210)
    x = rng.standard_normal((B, E), dtype=np.float32) * np.float32(4.0)
    hist = rng.integers(0, V, (B, LASTN)).astype(np.int32)
    seeds = qa.gen_row_seeds(19, 0, B)
    bats = [qa.Batch(B, V, LASTN) for _ in range(2)]
    dwr, dx = qa.DeviceBuffer.from_array(wq), qa.DeviceBuffer.from_array(x)
    w_bytes = qa.head_exact_packed_bytes(WT, E, V)
    dw = qa.DeviceBuffer(w_bytes)
    bats[0].head_exact_pack(WT, dwr.ptr, E, V, dw.ptr)
    bats[0].synchronize()
    dwr.free()
    dl, dl2 = qa.DeviceBuffer(4 * B * V), qa.DeviceBuffer(4 * B * V)
    for bt in bats:
        bt.config(0, B, T, TOPP, K, MINP, RP, LASTN, seeds=seeds)
        bt.set_history(0, hist)
    orc = Oracle()
    ids_f = bats[0].pick_head_exact(WT, dw.ptr, dx.ptr, E, B, V, dl.ptr)
    logits = dl.download(np.float32, B * V).reshape(B, V)
    want = orc.head_gemv(WT, wq, x, V, n_threads=min(16, os.cpu_count() or 1))
    nan_g, nan_w = np.isnan(logits), np.isnan(want)
    logit_mism = int(np.count_nonzero(nan_g != nan_w)) + int(np.count_nonzero(
        logits.view(np.uint32)[~nan_g & ~nan_w] != want.view(np.uint32)[~nan_g & ~nan_w]))
    dl2.upload(logits)
    ids_p = bats[1].pick(dl2.ptr, V, B, V)
    mism = int((ids_f != ids_p).sum())
    mism += sum(int(bats[0].get_state(r)[0] != bats[1].get_state(r)[0]) for r in range(B))
    cpu_mism = 0
    for r in range(B):
        smp = orc.sampler()
        smp.config(T, TOPP, K, MINP, RP, LASTN, seed=int(seeds[r]))
        smp.set_history(hist[r])
        cpu_mism += int(smp.pick(want[r]) != int(ids_f[r]))
    # the CPU path: the restatement's gemv of one row on one core and its sampler
    smp = orc.sampler()
    t0, n_cpu = time.perf_counter(), 0
    while n_cpu < 3 or time.perf_counter() - t0 < 6.0:
        row = orc.head_gemv(WT, wq, x[n_cpu % B][None, :], V, n_threads=1)[0]
        smp.config(T, TOPP, K, MINP, RP, LASTN, seed=1 + n_cpu)
        smp.pick(row)
        n_cpu += 1
    cpu_rate = n_cpu / (time.perf_counter() - t0)
    bats[0].time_head_exact(WT, dw.ptr, dx.ptr, E, B, V, dl.ptr, max(args.warmup, 20), 1)
    res = {}
    for name, mode in (("fused", 1), ("unfused", 0), ("layer_alone", 2)):
        bats[0].time_head_exact(WT, dw.ptr, dx.ptr, E, B, V, dl.ptr, 5, mode)
        res[name] = bats[0].time_head_exact(WT, dw.ptr, dx.ptr, E, B, V, dl.ptr, args.steps,
                                            mode) * 1e3 / args.steps
    layer_bytes = w_bytes + 4 * B * E + 4 * B * V
    us_layer = res["layer_alone"]
    gbs = layer_bytes / (us_layer * 1e-6) / 1e9
    # the reference's arithmetic per weight: a byte to float, the scale product, then per row
    # a product and a sum (2 + 2 B operations), against 256 CUs x 4 SIMDs x 16 lanes at
    # 2.4 GHz (39.3e12 unpacked lane operations per second: the 157.3 TFLOP/s fp32 peak
    # counts an FMA as two and packed pairs as two)
    valu_ops = float(V) * E * (2 + 2 * B)
    valu_peak = 256 * 4 * 16 * 2.4e9
    print(json.dumps({
        "metric": "exact output layer + pick rows/s (fused epilogue)",
        "value": B / (res["fused"] * 1e-6), "unit": "rows/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": res["fused"] / 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"lm_head_exact_b{B}", "rows": B, "n_embd": E, "vocab": V,
                   "weight_type": "Q6_K", "top_k": K, "temperature": T, "top_p": TOPP,
                   "min_p": MINP, "repeat_penalty": RP, "last_n": LASTN},
        "us": {k: round(v, 2) for k, v in res.items()},
        "roofline": {"kernel": "k_head_exact (layer alone)", "bound": "hbm",
                     "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": gbs / HBM_PEAK_GBS, "traffic": None,
                     "valu_frac": valu_ops / (us_layer * 1e-6) / valu_peak},
        "cpu_baseline": {"value": cpu_rate, "unit": "rows/s", "cores": 1, "kind": "port",
                         "sample": f"{n_cpu} rows: the restatement of forward_cpu.c's gemv "
                                   "(Q6_K rows dequantized, float sums in k order) on one "
                                   "core, then the restatement of sample.c"},
        "parity": {"rows": B, "logit_mismatches": logit_mism,
                   "fused_vs_unfused_mismatches": mism, "fused_vs_cpu_id_mismatches": cpu_mism}
    }), flush=True)
    for b_ in (dx, dw, dl, dl2):
        b_.free()
    for bt in bats:
        bt.close()


def sample_h_bench(args):
    """quasar_sampler_pick as the reference's server calls it once per token: host logits
    (pageable memory) in, one id out.  Each call copies the row to the device, picks, waits
    and copies the id back; timed one call at a time on the host clock after a warm-up.
    The parts are timed on their own as well: the row's copy to the device, the device
    pick of one row (events on the stream, back to back), and a 4-byte copy back."""
    import quasar_amd as qa
    from quasar_amd.workloads import STRESS, WORKLOADS
    w = dict(WORKLOADS, **STRESS)[args.workload or "full_b1"]
    V = w.vocab
    dbuf = qa.DeviceBuffer(4 * V)
    qa.gen_logits_device(dbuf, V, 0, 1, V, w.dist, w.sigma, w.boost, w.seed)
    host = dbuf.download(np.float32, V)
    smp = qa.Sampler()
    smp.config(*w.params(), seed=int(qa.gen_row_seeds(w.seed, 0, 1)[0]))
    for _ in range(max(args.warmup, 50)):
        smp.pick(host)
    n = max(args.steps, 100)
    lat = np.empty(n)
    for i in range(n):
        t0 = time.perf_counter_ns()
        smp.pick(host)
        lat[i] = (time.perf_counter_ns() - t0) / 1e3
    h2d = np.empty(n)
    for i in range(n):
        t0 = time.perf_counter_ns()
        dbuf.upload(host)
        h2d[i] = (time.perf_counter_ns() - t0) / 1e3
    d2h = np.empty(n)
    for i in range(n):
        t0 = time.perf_counter_ns()
        dbuf.download(np.int32, 1)
        d2h[i] = (time.perf_counter_ns() - t0) / 1e3
    bt = qa.Batch(1, V, max(1, w.repeat_last_n))
    bt.config(0, 1, *w.params(), seeds=[1])
    bt.time_picks([dbuf.ptr], V, 1, V, 200)
    dev_us = 1e3 * bt.time_picks([dbuf.ptr], V, 1, V, 1000) / 1000
    bt.close()
    smp.close()
    dbuf.free()
    q = lambda a: {"median": round(float(np.median(a)), 2), "p10": round(float(np.percentile(a, 10)), 2),
                   "p90": round(float(np.percentile(a, 90)), 2)}
    print(json.dumps({
        "metric": "sample.h quasar_sampler_pick latency (host logits in, id out)",
        "value": float(np.median(lat)), "unit": "us", "n_gpus": 1, "steps": n,
        "warmup": max(args.warmup, 50), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": w.name, "vocab": V, "row_bytes": 4 * V,
                   "description": w.description},
        "call_us": q(lat), "copy_in_us": q(h2d), "id_copy_out_us": q(d2h),
        "device_pick_us_back_to_back": round(dev_us, 2)}), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}): the sampler's "
              "rows are independent, so a multi-GPU run is B/G rows per GPU with no "
              "exchange; run it per GPU.", file=sys.stderr)
        sys.exit(2)
    if args.calibrate_copy:
        return calibrate_copy(args)
    if args.router:
        return router_bench(args)
    if args.head:
        return head_bench(args)
    if args.head_exact:
        return head_exact_bench(args)
    if args.sample_h:
        return sample_h_bench(args)
    import quasar_amd as qa
    from quasar_amd.workloads import BENCH_WORKLOAD, STRESS, WORKLOADS

    allw = dict(WORKLOADS, **STRESS)
    w = allw[args.workload or BENCH_WORKLOAD]
    wname = w.name
    if args.rows > 0 and args.rows != w.batch:
        w = w.with_batch(args.rows)
        wname = f"{w.name} settings at batch {args.rows}"
    B, V = w.batch, w.vocab
    dev_name, dev_mem, dev_cu = qa.device_info()
    dev_name = device_name(dev_name, dev_cu, dev_mem)
    print(f"# device {dev_name}, {dev_mem / 2**30:.0f} GiB, {dev_cu} CUs; workload {w.name}",
          file=sys.stderr, flush=True)

    nbytes = 4 * B * V
    n_buf = args.buffers or max(1, -(-CACHE_DEFEAT_BYTES // nbytes))
    bufs = []
    for _ in range(n_buf):
        bufs.append(qa.DeviceBuffer(nbytes))
        qa.gen_logits_device(bufs[-1], V, 0, B, V, w.dist, w.sigma, w.boost, w.seed)
    logits = bufs[0]
    seeds = qa.gen_row_seeds(w.seed, 0, B)
    hist = qa.gen_history(w.seed, 0, B, w.hist_len, V, w.hist_pool) if w.hist_len else None
    batch = qa.Batch(B, V, max(1, w.repeat_last_n))
    batch.set_mode({"auto": qa.MODE_AUTO, "split": qa.MODE_SPLIT,
                    "stream": qa.MODE_STREAM, "row": qa.MODE_ROW}[args.mode])
    batch.config(0, B, *w.params(), seeds=seeds)
    if hist is not None:
        batch.set_history(0, hist)

    used = MODE_NAMES.get(batch.resolve_mode(logits.ptr, V, B, V), "split")
    first_ids, diag = batch.pick(logits.ptr, V, B, V, diag=True)
    paths, fallbacks = {}, {}
    for d in diag:
        paths[d.path] = paths.get(d.path, 0) + 1
        if d.fallback:
            fallbacks[d.fallback] = fallbacks.get(d.fallback, 0) + 1

    # the GPU is timed first; the CPU baseline (seconds of host work, the GPU idle) after
    host = None if args.no_cpu else logits.download(np.float32, B * V).reshape(B, V)

    ptrs = [b.ptr for b in bufs]
    # untimed picks until the GPU has worked for --settle-s: after input generation it sits
    # at idle clocks, and the few warm-up steps of a short run do not bring it up
    settle_picks, settle_t0 = 0, time.perf_counter()
    while time.perf_counter() - settle_t0 < args.settle_s:
        batch.time_picks(ptrs, V, B, V, 20)
        settle_picks += 20
    for i in range(args.warmup):
        batch.pick_async(ptrs[i % n_buf], V, B, V)
    qa.check(qa.load().qs_device_synchronize(), "sync")
    t0 = time.perf_counter()
    ms = batch.time_picks(ptrs, V, B, V, args.steps)
    qa.check(qa.load().qs_device_synchronize(), "sync")
    wall = time.perf_counter() - t0

    ms_per_step = ms / args.steps
    rows_per_s = B / (ms_per_step * 1e-3)
    alg_bytes = B * w.algorithmic_bytes_per_row()
    pick_frac = alg_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS
    kernel_ms, kernel = ms_per_step, f"one pick ({KERNELS[used]})"
    kernel_ms_isolated = None
    if used == "row":
        # the row kernel is the whole pick, one launch a step: the timed region's events over
        # the back-to-back launches give its average duration (a kernel trace of the same run
        # shows each launch starting as the previous one ends)
        kernel = "k_row (the row kernel: the whole pick, launches back to back)"
        if args.kernel_steps > 0:
            kernel_ms_isolated = (batch.time_stream_kernel(ptrs, V, B, V, args.kernel_steps)
                                  / args.kernel_steps)
    elif used == "stream" and args.kernel_steps > 0:
        kernel_ms = batch.time_stream_kernel(ptrs, V, B, V, args.kernel_steps) / args.kernel_steps
        kernel = "k_part (the streaming kernel; k_decide follows it)"
    achieved = alg_bytes / (kernel_ms * 1e-3) / 1e9
    # the row pick's loads alone at its launch shape: the read ceiling of the same bytes
    read = None
    if used == "row" and B <= dev_cu:
        qa.time_row_reads(ptrs, V, B, V, 50)
        read_ms = qa.time_row_reads(ptrs, V, B, V, args.steps) / args.steps
        read_gbs = 4 * B * V / (read_ms * 1e-3) / 1e9
        read = {"kernel": "k_row_read (the row kernel's launch shape, chunks and loads, "
                          "adding the rows up and nothing else)",
                "ms": read_ms, "achieved": read_gbs, "unit": "GB/s",
                "frac": read_gbs / HBM_PEAK_GBS, "pick_over_read": ms_per_step / read_ms}
    traffic = committed_traffic(w.name, used) if wname == w.name else None
    cpu = None
    parity = None
    if host is not None:
        cpu, parity = cpu_baseline(w, host, hist, seeds, first_ids, diag, args)
        del host
    out = {
        "metric": METRIC.format(B=B, V=V),
        "value": rows_per_s,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": wname, "batch": B, "vocab": V, "history": w.hist_len,
                   "temperature": w.temperature, "top_k": w.top_k, "top_p": w.top_p,
                   "min_p": w.min_p, "repeat_penalty": w.repeat_penalty,
                   "mode": args.mode, "kernels": used, "input_buffers": n_buf,
                   "input_bytes_total": n_buf * nbytes, "settle_picks": settle_picks,
                   "description": w.description},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "traffic": traffic["bytes"] if traffic else None,
                     "traffic_source": traffic["source"] if traffic else None,
                     "kernel": kernel, "kernel_ms": kernel_ms,
                     "kernel_ms_isolated": kernel_ms_isolated, "pick_frac": pick_frac,
                     "bytes_per_step": alg_bytes},
        "read_ceiling": read,
        "cpu_baseline": cpu,
        "parity": parity,
        "paths": {str(k): v for k, v in sorted(paths.items())},
        "fallbacks": {str(k): v for k, v in sorted(fallbacks.items())},
        "wall_s_timed": wall,
        "device": dev_name,
    }
    print(json.dumps(out), flush=True)
    batch.close()
    for b_ in bufs:
        b_.free()


def device_name(name, n_cu, mem):
    """The device's name, else rocminfo's marketing name for the first GPU agent, else its
    architecture with its CU count and memory (some runtimes report no marketing name)."""
    if name and not name.startswith(" "):
        return name
    arch = name.strip(" ()") or "unknown architecture"
    fallback = f"{arch}, {n_cu} CUs, {mem / 2**30:.0f} GiB (no marketing name reported)"
    import shutil
    import subprocess
    tool = shutil.which("rocminfo") or "/opt/rocm/bin/rocminfo"
    try:
        txt = subprocess.run([tool], capture_output=True, text=True, timeout=60).stdout
    except (OSError, subprocess.SubprocessError):
        return fallback
    agent = ""
    for line in txt.splitlines():
        line = line.strip()
        if line.startswith("Name:"):
            agent = line.split(":", 1)[1].strip()
        elif line.startswith("Marketing Name:") and agent.startswith("gfx"):
            market = line.split(":", 1)[1].strip()
            return f"{market} ({agent})" if market else fallback
    return fallback


if __name__ == "__main__":
    main()
