"""Benchmark of the speculative-decoding verification path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config h|c1|c2|c3|c4|c5|v2]

A step is one ``rejection_sample`` call (the persistent verify kernel; with top-k / top-p the
constraints kernel before it) over the whole batch, inputs already resident in HBM; the
default workload is the headline configuration (B=256, k=4, V=151936, fp32 target logits and
draft probs, random T=0.8).  Prints ONE JSON line:

* value = GB/s over the bytes the kernel's algorithm moves (every verify row of the target
  once, plus target, draft and noise of each request's first rejected row, the decision
  inputs, metadata and output; from the run's own output, ``configs.kernel_bytes``) per step,
  step time over the timed region, which holds only the calls;
* config.reference_algorithm_bytes = the bytes the reference algorithm reads (every row
  scored, the survey's count), with the step rate on those bytes beside it;
* verified tokens/s, the accept-length histogram and per-position accept rates;
* roofline: kernel time from HIP events recorded around every launch on the launch stream, in
  a second pass of the same number of steps; traffic from the committed rocprofv3 summary when
  it was measured on the current kernel sources (their sha256), else null;
* cpu_baseline: the oracle (the reference algorithm on torch-CPU) on all host threads and on
  one, with each run-to-run spread; parity: the GPU tokens against that oracle run.

``--pmc-driver`` runs a 1 GiB device copy (the calibration kernel for rocprofv3 counters)
followed by a few headline steps, and prints nothing else; profiles/ records the rocprofv3
commands that use it.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "vllm-from-scratch_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402
import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0
TRAFFIC_FILE = ROOT / "profiles" / "verify_kernel_headline_traffic.md"


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="h", choices=["h", "c1", "c2", "c3", "c4", "c5", "v2"])
    ap.add_argument("--cpu-seconds", type=float, default=8.0,
                    help="minimum CPU time of each CPU-baseline sample (all threads, one thread)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--pmc-driver", action="store_true",
                    help="run the counter-calibration copy and a few steps, print nothing")
    return ap.parse_args()


def make_workload(name, device):
    from mvsd.testing import configs

    return {"h": configs.headline, "c1": configs.greedy_c1, "c2": configs.random_c2,
            "c4": configs.ragged_c4, "c5": configs.eagle_c5}[name](device)


def run_step(w):
    """One verification step: rejection_sample on the raw target rows with the temperature
    divide and, for workloads with top-k / top-p (c4), the sampling constraints applied in the
    kernels (RejectionSampler.forward's path when no penalty needs the processed rows)."""
    from mvsd.sample.metadata import SamplingMetadata
    from mvsd.sample.rejection_sampler import rejection_sample

    sm = SamplingMetadata(temperature=w.temperature, all_greedy=w.all_greedy,
                          all_random=w.all_random, top_k=w.top_k, top_p=w.top_p)
    constrained = w.top_k is not None or w.top_p is not None

    def step():
        return rejection_sample(
            w.draft_token_ids, w.num_draft_tokens, w.max_spec_len, w.cu_num_draft_tokens,
            w.draft_probs, w.target_logits, w.bonus_token_ids, sm, uniform_probs=w.uniforms,
            exp_noise=w.exp_noise, target_rows=w.target_rows,
            apply_temperature=w.apply_temperature or constrained,
            apply_top_k_top_p=constrained)
    return step


def settle_gpu(seconds=0.1):
    """Bring the GPU out of its idle clock state before the warm-up steps: device-to-device
    copies of a 256 MiB buffer for `seconds` (not the workload; nothing from it is kept).
    Without it the first tens of timed steps of a fresh process run a few percent slower."""
    a = torch.empty(64 << 20, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(10):
            b.copy_(a)
        torch.cuda.synchronize()
    del a, b
    torch.cuda.synchronize()


LAUNCH_MEDIAN_MS = [0.0]  # median of the last time_steps call's per-call event times


def time_steps(step, steps, warmup):
    """Time `steps` calls after `warmup` untimed ones.  Returns (ms per step over the timed
    region, mean ms between HIP events recorded right before and after each call, wall ms per
    step, last output); the median of the per-call event times goes to LAUNCH_MEDIAN_MS[0].  The timed region holds only the calls, between two events; the
    per-call events are recorded in a second pass of `steps` calls, so that their markers do
    not inflate the timed region.  All events are recorded on the current stream, the stream
    the kernels are launched on."""
    settle_gpu()
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        out = step()
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    total = start.elapsed_time(end) / steps
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(2 * steps)]
    for i in range(steps):
        marks[2 * i].record(stream)
        step()
        marks[2 * i + 1].record(stream)
    torch.cuda.synchronize()
    per = [marks[2 * i].elapsed_time(marks[2 * i + 1]) for i in range(steps)]
    LAUNCH_MEDIAN_MS[0] = float(np.median(per))
    return total, float(np.mean(per)), wall / steps * 1e3, out


def accept_histogram(outputs, num_draft_tokens, max_k):
    hist = [0] * (max_k + 1)
    for toks, k in zip(outputs, num_draft_tokens):
        if k > 0:
            hist[max(len(toks) - 1, 0)] += 1
    return hist


def cpu_oracle_runner(w):
    """A callable running the CPU oracle (oracle/rejection.py on torch-CPU, the reference's
    algorithm step by step) over the whole workload on host copies of the same inputs,
    uniforms and noise; with top-k / top-p, the processed path (temperature, constraints, then
    verification)."""
    from oracle import rejection as orc

    ks = w.num_draft_tokens
    rows = w.target_rows.long() if w.target_rows is not None else None
    tl = (w.target_logits if rows is None else w.target_logits[rows]).cpu()
    dp = None if w.draft_probs is None else w.draft_probs.cpu()
    noise = None if w.exp_noise is None else w.exp_noise.cpu()
    u = None if w.uniforms is None else w.uniforms.cpu()
    temp = None if w.temperature is None else w.temperature.cpu()
    ids = w.draft_token_ids.cpu()
    bonus = w.bonus_token_ids.cpu()

    constrained = w.top_k is not None or w.top_p is not None
    if constrained:
        from oracle import topk_topp as otp

        req = torch.from_numpy(orc.request_of_row(ks))
        row_t = temp[req]
        row_t = torch.where(row_t == 0, torch.ones_like(row_t), row_t)
        row_k = None if w.top_k is None else w.top_k.cpu()[req]
        row_p = None if w.top_p is None else w.top_p.cpu()[req]

    def run():
        if constrained:
            x = otp.apply_top_k_top_p(tl.float() / row_t.unsqueeze(-1), row_k, row_p)
            return orc.rejection_sample(ids, ks, w.max_spec_len, dp, x, bonus, temperature=temp,
                                        all_greedy=w.all_greedy, uniforms=u, exp_noise=noise,
                                        apply_temperature=False)
        return orc.rejection_sample(ids, ks, w.max_spec_len, dp, tl, bonus, temperature=temp,
                                    all_greedy=w.all_greedy, uniforms=u, exp_noise=noise,
                                    apply_temperature=w.apply_temperature)
    return run


def cpu_baseline(w, min_seconds):
    """Time the CPU oracle on all host threads, then on one thread, each repeated until at
    least `min_seconds` of CPU work; GB/s over the reference algorithm's bytes.  Returns the
    cpu_baseline object (all threads, with the one-thread figure and the run-to-run spread of
    both) and the oracle's result for the parity check."""
    from mvsd.testing import configs

    run = cpu_oracle_runner(w)
    nbytes = configs.algorithmic_bytes(w)
    all_threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    figures = []
    ref = None
    for threads in (all_threads, 1):
        torch.set_num_threads(threads)
        ref = run()  # warm-up (and the parity reference)
        times = []
        t0 = time.perf_counter()
        while True:
            t1 = time.perf_counter()
            run()
            times.append(time.perf_counter() - t1)
            if time.perf_counter() - t0 >= min_seconds:
                break
        rates = [nbytes / t / 1e9 for t in times]
        figures.append({"cores": threads, "value": round(nbytes * len(times) / sum(times) / 1e9, 3),
                        "min": round(min(rates), 3), "max": round(max(rates), 3),
                        "runs": len(times), "seconds": round(sum(times), 2)})
    torch.set_num_threads(all_threads)
    main = figures[0]
    return {"value": main["value"], "unit": "GB/s", "cores": main["cores"], "kind": "port",
            "sample": f"the whole workload ({w.batch_size} requests, {w.num_tokens} verify rows, "
                      f"V={w.vocab_size}) through oracle/rejection.py on torch-CPU (the "
                      f"reference algorithm: every row scored), repeated back to back after one "
                      f"warm-up, on {main['cores']} threads and on 1; GB/s over the reference "
                      f"algorithm's bytes; min/max are the per-run spread; inputs in host "
                      f"memory, same uniforms and noise as the GPU run",
            "by_cores": figures}, ref


# Sources whose change invalidates a committed counter summary of the verify kernel.
# The sources the headline's verify launch is built and planned from (the constraints kernel
# does not run at the headline).
KERNEL_SOURCES = ["vllm-from-scratch_amd/csrc/verify.hip", "vllm-from-scratch_amd/csrc/verify.h",
                  "vllm-from-scratch_amd/csrc/capi.hip", "vllm-from-scratch_amd/csrc/mvsd_device.h"]


def kernel_sources_sha256():
    import hashlib

    h = hashlib.sha256()
    for rel in KERNEL_SOURCES:
        h.update((ROOT / rel).read_bytes())
    return h.hexdigest()


def load_traffic(config):
    """HBM bytes per launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary (a
    line ``traffic_bytes_per_launch[<config>] = N``), used only when the summary's
    ``kernel_sources_sha256`` matches the current kernel sources; else None."""
    if not TRAFFIC_FILE.exists():
        return None
    value, sha = None, None
    key = f"traffic_bytes_per_launch[{config}] = "
    for line in TRAFFIC_FILE.read_text().splitlines():
        if line.startswith(key):
            value = int(line[len(key):].strip())
        if line.startswith("kernel_sources_sha256 = "):
            sha = line.split("=", 1)[1].strip()
    if value is None or sha != kernel_sources_sha256():
        return None
    return value


def bench_ngram(args, device):
    from mvsd.spec_decode.ngram_proposer_gpu import ngram_propose_device
    from mvsd.testing import configs
    from oracle import ngram as ong

    tokens = configs.ngram_c3(device)
    B, L = tokens.shape
    lens = torch.full((B,), L, dtype=torch.int32, device=device)

    def step():
        return ngram_propose_device(tokens, lens, min_n=2, max_n=5, k=5)

    ms, _, wall_ms, (d, v) = time_steps(step, args.steps, args.warmup)
    nbytes = B * L * 4 + B * 4 + B * 5 * 4 + B * 4
    tn, ln = tokens.cpu().numpy(), lens.cpu().numpy()
    t0 = time.perf_counter()
    ong.kmp_batch(tn, ln, 2, 5, 8192, 5)
    cpu_s = time.perf_counter() - t0
    host_ms = bench_ngram_host_api(tn, ln, args.steps, args.warmup, device)
    line = {"metric": "ngram proposer drafts/s (C3)", "value": round(B / (ms / 1e3), 1),
            "unit": "requests/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "strong",
            "vs_baseline": None, "dtype": "int32", "data": "synthetic",
            "config": {"workload": "c3 ngram B=256 L=4096 min_n=2 max_n=5 k=5"},
            "roofline": {"bound": "hbm", "achieved": round(nbytes / (ms / 1e3) / 1e9, 2),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(nbytes / (ms / 1e3) / 1e9 / HBM_PEAK_GBS, 5),
                         "traffic": None},
            "cpu_baseline": {"value": round(B / cpu_s, 1), "unit": "requests/s", "cores": 1,
                             "kind": "port", "sample": "all 256 histories through oracle/ngram.c "
                             "KMP (the reference CPU algorithm), one thread"},
            "host_api": {"ms_per_call": round(host_ms, 5),
                         "requests_per_s": round(B / (host_ms / 1e3), 1),
                         "path": "NgramProposer.propose on pageable numpy histories [256, 4096] "
                                 "int32: pinned staging, one upload, the kernel, drafts and "
                                 "counts back, one synchronisation (wall clock)"}}
    print(json.dumps(line))


def bench_ngram_host_api(tokens_np, lens_np, steps, warmup, device):
    """Wall-clock ms per NgramProposer.propose call (the reference's host-buffer API) on the
    C3 histories held in pageable host memory."""
    from types import SimpleNamespace

    from mvsd.spec_decode.ngram_proposer import NgramProposer

    B = tokens_np.shape[0]
    cfg = SimpleNamespace(
        speculative_config=SimpleNamespace(num_speculative_tokens=5, prompt_lookup_min=2,
                                           prompt_lookup_max=5),
        model_config=SimpleNamespace(max_model_len=8192),
        scheduler_config=SimpleNamespace(max_num_seqs=B))
    prop = NgramProposer(cfg, device)
    sampled = [[1]] * B
    for _ in range(warmup):
        prop.propose(5, sampled, lens_np, tokens_np)
    t0 = time.perf_counter()
    for _ in range(steps):
        prop.propose(5, sampled, lens_np, tokens_np)
    return (time.perf_counter() - t0) / steps * 1e3


def bench_v2(args, device):
    """The V2 runner's verification (mvsd.worker.gpu.spec_decode.rejection_sample) on the
    headline shape: B=256, k=4, V=151936 fp32, all random at T=0.8, draft logits
    [B, k, V] pre-temperature, target = draft + N(0, 0.5^2) (already scaled), drafts sampled
    from softmax(draft / T), 1280 target rows (each request's 4 verify rows and its bonus
    row).  Algorithmic bytes = verify rows of target and draft once + the bonus rows that are
    resampled + the index arrays and outputs."""
    from mvsd.worker.gpu.spec_decode import rejection_sample
    from oracle import v2_rejection as ov2

    B, K, V, T = 256, 4, 151936, 0.8
    g = torch.Generator(device=device).manual_seed(2002)
    draft = torch.randn(B, K, V, generator=g, device=device) * 2.0
    rows = B * (K + 1)
    target = torch.empty(rows, V, device=device)
    tv = target.view(B, K + 1, V)
    tv[:, :K] = draft + 0.5 * torch.randn(B, K, V, generator=g, device=device)
    tv[:, K] = torch.randn(B, V, generator=g, device=device) * 2.0
    probs = torch.softmax(draft.view(B * K, V) / T, -1)
    ids = torch.multinomial(probs, 1, generator=g).view(B, K).to(torch.int32)
    del probs
    ds = torch.zeros(B, K + 1, dtype=torch.int32, device=device)
    ds[:, 1:] = ids
    ar = torch.arange(B, dtype=torch.int32, device=device)
    case = dict(target_logits=target, draft_logits=draft, draft_sampled=ds.view(-1),
                cu_num_logits=torch.arange(0, rows + 1, K + 1, dtype=torch.int32, device=device),
                pos=torch.arange(rows, dtype=torch.int64, device=device) + 4096,
                idx_mapping=ar, expanded_idx_mapping=ar.repeat_interleave(K + 1),
                expanded_local_pos=torch.arange(K + 1, dtype=torch.int32,
                                                device=device).repeat(B),
                temperature=torch.full((B,), T, device=device),
                seed=torch.randint(0, 2**62, (B,), generator=g, device=device),
                num_speculative_steps=K)
    torch.cuda.synchronize()

    def step():
        return rejection_sample(**case)

    ms, launch_ms, wall_ms, (s, n) = time_steps(step, args.steps, args.warmup)
    n_host = n.cpu().numpy()
    n_bonus = int((n_host == K + 1).sum())
    P = B * K
    nbytes = 2 * P * V * 4 + n_bonus * V * 4 + rows * (4 + 8 + 4 + 4) + B * (4 + 4 + 4 + 8) \
        + B * (K + 1) * 8 + B * 4
    hist = np.bincount(n_host - 1, minlength=K + 1).tolist()
    gbs = nbytes / (ms / 1e3) / 1e9
    kernel_gbs = nbytes / (launch_ms / 1e3) / 1e9
    line = {"metric": "V2 rejection-sampler HBM GB/s (% of peak) + verified tok/s, B=256 k=4 V=152k",
            "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "f32",
            "data": "synthetic (seeded torch generator on device; no checkpoint)",
            "config": {"workload": "v2 B=256 k=4 V=151936 fp32 random T=0.8, draft logits",
                       "batch_size": B, "num_logits": rows, "vocab_size": V,
                       "algorithmic_bytes": nbytes},
            "pct_of_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
            "verified_tok_per_s": round(float(n_host.sum()) / (ms / 1e3), 1),
            "accept_length_hist": hist, "wall_ms_per_step": round(wall_ms, 5),
            "roofline": {"bound": "hbm", "achieved": round(kernel_gbs, 2), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(kernel_gbs / HBM_PEAK_GBS, 4),
                         "traffic": None,
                         "kernel": "v2_stats + v2_chain + v2_resample + v2_insert per call",
                         "kernel_ms": round(launch_ms, 5),
                         "kernel_ms_median": round(LAUNCH_MEDIAN_MS[0], 5)},
            "cpu_baseline": None}
    if not args.no_cpu_baseline:
        sub = 16  # requests in the CPU sample
        host = {k: (v.cpu().numpy() if isinstance(v, torch.Tensor) else v)
                for k, v in case.items()}
        r_rows = sub * (K + 1)
        host["target_logits"] = host["target_logits"][:r_rows]
        for k in ("draft_sampled", "pos", "expanded_idx_mapping", "expanded_local_pos"):
            host[k] = host[k][:r_rows]
        host["cu_num_logits"] = host["cu_num_logits"][:sub + 1]
        host["idx_mapping"] = host["idx_mapping"][:sub]
        t0 = time.perf_counter()
        runs = 0
        while True:
            es, en = ov2.rejection_sample(**host)
            runs += 1
            if time.perf_counter() - t0 >= min(args.cpu_seconds, 10.0):
                break
        cpu_s = (time.perf_counter() - t0) / runs
        ok = bool((en == n_host[:sub]).all())
        sub_bytes = nbytes * sub / B
        line["cpu_baseline"] = {"value": round(sub_bytes / cpu_s / 1e9, 4), "unit": "GB/s",
                                "cores": 1, "kind": "port",
                                "sample": f"first {sub} of {B} requests through "
                                f"oracle/v2_rejection.py (numpy), {runs} runs; "
                                f"num_sampled equal to the GPU's: {ok}",
                                "seconds": round(cpu_s * runs, 2)}
    print(json.dumps(line), flush=True)


def main():
    args = parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 "
                          "(request or vocabulary sharding across GPUs is not launched)"}))
        sys.exit(2)
    device = torch.device("cuda", 0)
    if args.config == "c3":
        bench_ngram(args, device)
        return
    if args.config == "v2":
        bench_v2(args, device)
        return
    from mvsd.sample.rejection_sampler import RejectionSampler
    from mvsd.testing import configs

    w = make_workload(args.config, device)
    step = run_step(w)
    if args.pmc_driver:
        a = torch.empty(256 * 1024 * 1024, dtype=torch.float32, device=device)  # 1 GiB
        b = torch.empty_like(a)
        b.copy_(a)
        torch.cuda.synchronize()
        del a, b
        for _ in range(3):
            step()
        torch.cuda.synchronize()
        return
    ms, launch_ms, wall_ms, out = time_steps(step, args.steps, args.warmup)
    outputs, _ = RejectionSampler.parse_output(out, w.vocab_size)
    constrained = w.top_k is not None or w.top_p is not None
    # the constraints kernel reads each constrained row about twice (top-k: one pass and an
    # LDS selection; top-p: a histogram pass and a gather pass), counted as two passes
    nbytes = configs.kernel_bytes(w, outputs, constrained_passes=2 if constrained else 0)
    ref_bytes = configs.algorithmic_bytes(w)
    tokens = sum(len(o) for o in outputs)
    gbs = nbytes / (ms / 1e3) / 1e9
    kernel_gbs = nbytes / (launch_ms / 1e3) / 1e9
    hist = accept_histogram(outputs, w.num_draft_tokens, w.max_spec_len)
    line = {
        "metric": "rejection-sampler HBM GB/s (% of peak) + verified tok/s, B=256 k=4 V=152k",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if w.target_logits.dtype == torch.float32 else "bf16",
        "data": "synthetic (seeded on-device Philox; random logits, no checkpoint)",
        "config": {"workload": {"h": "headline B=256 k=4 V=151936 fp32 random T=0.8",
                                "c1": "c1 greedy B=4 k=3 fp32", "c2": "c2 random B=64 k=4 fp32",
                                "c4": "c4 ragged B=512 bf16, top-k=50 / top-p=0.9 quartiles",
                                "c5": "c5 eagle B=1024 k=7 bf16 target"}[args.config],
                   "batch_size": w.batch_size, "num_draft_rows": w.num_tokens,
                   "vocab_size": w.vocab_size,
                   "kernel_bytes": nbytes,
                   "reference_algorithm_bytes": ref_bytes,
                   "effective_GBps_on_reference_bytes": round(ref_bytes / (ms / 1e3) / 1e9, 2)},
        "pct_of_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "verified_tok_per_s": round(tokens / (ms / 1e3), 1),
        "verified_tokens_per_step": tokens,
        "accept_length_hist": hist,
        "accept_rate_by_position": accept_rates(outputs, w.num_draft_tokens, w.max_spec_len),
        "wall_ms_per_step": round(wall_ms, 5),
        "roofline": {"bound": "hbm", "achieved": round(kernel_gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(kernel_gbs / HBM_PEAK_GBS, 4),
                     "traffic": load_traffic(args.config),
                     "kernel": ("mvsd::verify_kernel"
                                + (" + constraints_kernel" if constrained else "")
                                + " per rejection_sample"),
                     "kernel_ms": round(launch_ms, 5),
                     "kernel_ms_median": round(LAUNCH_MEDIAN_MS[0], 5)},
        "cpu_baseline": None,
        "parity": None,
    }
    if args.config == "h":
        line["drop_in_forward"] = bench_forward(w, args.steps, args.warmup)
    if not args.no_cpu_baseline:
        line["cpu_baseline"], ref = cpu_baseline(w, args.cpu_seconds)
        line["parity"] = parity_summary(w, out, ref)
    print(json.dumps(line), flush=True)


def bench_forward(w, steps, warmup):
    """ms per RejectionSampler.forward call (the drop-in's whole step) on the same rows in the
    compact [P + B, V] layout: bonus rows through mvsd.sample.Sampler, the uniforms and the
    [B, V] Exp(1) noise drawn by torch's generator, then the verification.  Reported beside
    the headline, which times rejection_sample with the randomness supplied."""
    from mvsd.sample import Sampler
    from mvsd.sample.rejection_sampler import RejectionSampler
    from mvsd.testing.spec_metadata import make_metadata, sampling_metadata

    B, P, V = w.batch_size, w.num_tokens, w.vocab_size
    ids = w.draft_token_ids.tolist()
    drafts, start = [], 0
    for k in w.num_draft_tokens:
        drafts.append(ids[start:start + k])
        start += k
    device = w.target_logits.device
    meta = make_metadata(drafts, device=device)
    logits = torch.empty((P + B, V), dtype=torch.float32, device=device)
    logits[meta.target_logits_indices.long()] = w.target_logits
    logits[meta.bonus_logits_indices.long()] = w.target_logits[:B]
    temps = w.temperature.tolist()
    sm = sampling_metadata(temps, drafts, device=device)
    rs = RejectionSampler(Sampler())

    def step():
        return rs(meta, w.draft_probs, logits, sm).sampled_token_ids

    ms, _, wall_ms, _ = time_steps(step, steps, warmup)
    del logits
    return {"ms_per_step": round(ms, 5), "wall_ms_per_step": round(wall_ms, 5),
            "path": "RejectionSampler(Sampler()).forward on compact [P + B, V] fp32 logits: "
                    "bonus-row sampling, uniforms and Exp(1) noise from torch's generator, "
                    "verification (no penalties, no logprobs)"}


def accept_rates(outputs, num_draft_tokens, max_k):
    """Per draft position j: accepted / drafted over the requests with more than j drafts
    (the per-position counts of SpecDecodingStats.observe_draft)."""
    drafted = np.zeros(max_k, dtype=np.int64)
    accepted = np.zeros(max_k, dtype=np.int64)
    for toks, k in zip(outputs, num_draft_tokens):
        drafted[:k] += 1
        accepted[:max(len(toks) - 1, 0)] += 1
    return [round(float(a) / d, 4) if d else None for a, d in zip(accepted, drafted)]


def parity_summary(w, out, ref):
    """Token parity of the GPU output against the oracle's on the same inputs: requests whose
    output differs, and how many of those differ only at an acceptance margin below 1e-6 or a
    recovered-token near-tie (the allowances of the parity bar); anything else is
    `unexplained` and fails the tests."""
    from oracle import rejection as orc

    rep = orc.compare(out.cpu().numpy(), ref, w.draft_token_ids.cpu(), w.num_draft_tokens)
    return {"requests": rep.requests, "mismatched": rep.mismatched,
            "accept_flips": rep.accept_flips, "recovered_flips": rep.recovered_flips,
            "unexplained": len(rep.unexplained)}


if __name__ == "__main__":
    main()
