"""Benchmark of the speculative-decoding verification path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config h|c1|c2|c3|c4|c5|v2]
                    [--configs c1,c2,c3,c4,c5,v2 | none]

A step is one ``rejection_sample`` call (the persistent verify kernel; with top-k / top-p the
plan and constraints kernels before it) over the whole batch, inputs already resident in HBM;
the default workload is the headline configuration (B=256, k=4, V=151936, fp32 target logits
and draft probs, random T=0.8).  Prints ONE JSON line:

* value = GB/s over the bytes the kernel's algorithm moves (every verify row of the target
  once, plus target, draft and noise of each request's first rejected row, the decision
  inputs, metadata and output; from the run's own output, ``configs.kernel_bytes``) per step,
  step time = the timed region (K back-to-back calls between two HIP events on the launch
  stream) / K;
* config.reference_algorithm_bytes = the bytes the reference algorithm reads (every row
  scored), with the step rate on those bytes beside it;
* verified tokens/s, the accept-length histogram and per-position accept rates;
* roofline: the same timed region (the verify kernel is the step's only launch at the
  headline); traffic from the committed rocprofv3 summary when it was measured on the current
  kernel sources (their sha256), else null;
* cpu_baseline: the oracle (the reference algorithm on torch-CPU) on all host threads and on
  one, with each run-to-run spread; parity: the GPU tokens against that oracle run;
* drop_in_forward: ``RejectionSampler(Sampler()).forward`` on the compact logits (bonus rows
  sampled on the device, randomness from torch's generator);
* configs: the other BASELINE configurations measured the same way in the same run (C1
  greedy, C2 random, C3 ngram, C4 ragged with top-k / top-p, C5 EAGLE-style with its drop-in
  forward, and the V2 boundary), each with its step time, byte counts and fractions of peak,
  accept statistics, parity against the oracle on the same inputs (a stated request slice for
  C4 and C5) and a bounded CPU baseline on all threads and on one.

``--config X`` prints the line of configuration X alone.  ``--pmc-driver`` runs a 1 GiB device
copy (the calibration kernel for rocprofv3 counters) followed by a few steps of the chosen
configuration, and prints nothing else; profiles/ records the rocprofv3 commands that use it.
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
METRIC = "rejection-sampler HBM GB/s (% of peak) + verified tok/s, B=256 k=4 V=152k"
SUB_CONFIGS = ("c1", "c2", "c3", "c4", "c5", "v2")
WORKLOAD_NAMES = {"h": "headline B=256 k=4 V=151936 fp32 random T=0.8",
                  "c1": "c1 greedy B=4 k=3 V=151936 fp32",
                  "c2": "c2 random B=64 k=4 V=151936 fp32 T=0.8",
                  "c4": "c4 ragged B=512 K~U{0..8} V=151936 bf16, half greedy, T~U[0.3,1.5], "
                        "top-k=50 / top-p=0.9 quartiles",
                  "c5": "c5 eagle B=1024 k=7 V=151936 bf16 target, T=1"}
# Requests in the CPU-baseline sample and in the parity check of each verify configuration
# (None = the whole workload).  C4's oracle pipeline sorts every constrained row on the host
# and C5 holds 7168 verify rows, so both take a leading slice of their requests; requests are
# independent, so the oracle's result for a slice equals its result for those requests of the
# whole batch.
CPU_SAMPLE = {"h": None, "c1": None, "c2": None, "c4": 32, "c5": 128}
PARITY_SAMPLE = {"h": None, "c1": None, "c2": None, "c4": 128, "c5": 256}

# Sources whose change invalidates a committed counter summary, and the summary, per config.
_CSRC = "vllm-from-scratch_amd/csrc/"
VERIFY_SOURCES = [_CSRC + f for f in ("verify.hip", "verify.h", "capi.hip", "mvsd_device.h")]
TRAFFIC = {
    "h": (ROOT / "profiles" / "verify_kernel_headline_traffic.md", VERIFY_SOURCES),
    "c4": (ROOT / "profiles" / "constraints_and_verify_c4_traffic.md",
           VERIFY_SOURCES + [_CSRC + "constraints.hip"]),
    "c5": (ROOT / "profiles" / "verify_kernel_c5_traffic.md", VERIFY_SOURCES),
    "c1": (ROOT / "profiles" / "verify_kernel_c1_traffic.md", VERIFY_SOURCES),
    "c2": (ROOT / "profiles" / "verify_kernel_c2_traffic.md", VERIFY_SOURCES),
    "v2": (ROOT / "profiles" / "v2_verify_kernels_traffic.md",
           [_CSRC + f for f in ("v2_verify.hip", "verify.h", "mvsd_device.h")]),
    "c3": (ROOT / "profiles" / "ngram_kernel_c3_traffic.md",
           [_CSRC + f for f in ("ngram.hip", "rows.h", "mvsd_device.h")]),
}


def parse_args(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="h", choices=["h", *SUB_CONFIGS])
    ap.add_argument("--configs", default=",".join(SUB_CONFIGS),
                    help="configurations measured after the headline and reported under "
                         "'configs' (comma list, or 'none')")
    ap.add_argument("--sub-steps", type=int, default=20,
                    help="timed steps of each configuration under 'configs'")
    ap.add_argument("--cpu-seconds", type=float, default=8.0,
                    help="minimum CPU time of each headline CPU-baseline sample (all threads, "
                         "one thread)")
    ap.add_argument("--sub-cpu-seconds", type=float, default=2.5,
                    help="minimum CPU time of each CPU-baseline sample under 'configs'")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--pmc-driver", action="store_true",
                    help="run the counter-calibration copy and a few steps, print nothing")
    return ap.parse_args(argv)


def make_workload(name, device):
    from mvsd.testing import configs

    return {"h": configs.headline, "c1": configs.greedy_c1, "c2": configs.random_c2,
            "c4": configs.ragged_c4, "c5": configs.eagle_c5}[name](device)


def is_constrained(w) -> bool:
    return w.top_k is not None or w.top_p is not None


def run_step(w):
    """One verification step: rejection_sample on the raw target rows with the temperature
    divide and, for workloads with top-k / top-p (c4), the sampling constraints applied in the
    kernels (RejectionSampler.forward's path when no penalty needs the processed rows)."""
    from mvsd.sample.metadata import SamplingMetadata
    from mvsd.sample.rejection_sampler import rejection_sample

    sm = SamplingMetadata(temperature=w.temperature, all_greedy=w.all_greedy,
                          all_random=w.all_random, top_k=w.top_k, top_p=w.top_p)
    constrained = is_constrained(w)

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


def time_steps(step, steps, warmup):
    """Time `steps` calls after `warmup` untimed ones.  Returns (ms per step over the timed
    region, wall ms per step, last output).  The timed region holds only the calls, back to
    back, between two HIP events recorded on the current stream, the stream the kernels are
    launched on, after a synchronisation on both sides."""
    settle_gpu()
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    out = None
    for _ in range(steps):
        out = step()
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return start.elapsed_time(end) / steps, wall / steps * 1e3, out


def accept_histogram(outputs, num_draft_tokens, max_k):
    hist = [0] * (max_k + 1)
    for toks, k in zip(outputs, num_draft_tokens):
        if k > 0:
            hist[max(len(toks) - 1, 0)] += 1
    return hist


def accept_rates(outputs, num_draft_tokens, max_k):
    """Per draft position j: accepted / drafted over the requests with more than j drafts
    (the per-position counts of SpecDecodingStats.observe_draft)."""
    drafted = np.zeros(max_k, dtype=np.int64)
    accepted = np.zeros(max_k, dtype=np.int64)
    for toks, k in zip(outputs, num_draft_tokens):
        drafted[:k] += 1
        accepted[:max(len(toks) - 1, 0)] += 1
    return [round(float(a) / d, 4) if d else None for a, d in zip(accepted, drafted)]


def head(w, n):
    """Workload of the first n requests of w (w itself when n is None or covers it)."""
    from dataclasses import replace

    if n is None or n >= w.batch_size:
        return w
    ks = list(w.num_draft_tokens[:n])
    P = int(sum(ks))

    def cut(t, m):
        return None if t is None else t[:m]
    return replace(
        w, num_draft_tokens=ks, max_spec_len=w.max_spec_len,
        draft_token_ids=w.draft_token_ids[:P], cu_num_draft_tokens=w.cu_num_draft_tokens[:n],
        target_logits=w.target_logits if w.target_rows is not None else w.target_logits[:P],
        target_rows=cut(w.target_rows, P), draft_probs=cut(w.draft_probs, P),
        bonus_token_ids=w.bonus_token_ids[:n], temperature=cut(w.temperature, n),
        uniforms=cut(w.uniforms, P), exp_noise=cut(w.exp_noise, n), top_k=cut(w.top_k, n),
        top_p=cut(w.top_p, n))


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

    constrained = is_constrained(w)
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


def all_host_threads() -> int:
    return int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))


def time_on_threads(run, min_seconds, amount, digits=4):
    """Run `run(threads)` once as a warm-up, then back to back until `min_seconds` have passed,
    on all host threads and then on one.  Each figure is `amount` (GB, or requests) per second
    of a run, over the runs (`value`) and per run (`min`, `max`).  Returns ([figure per thread
    count], warm-up result)."""
    all_threads = all_host_threads()
    figures, first = [], None
    for threads in (all_threads, 1):
        torch.set_num_threads(threads)
        res = run(threads)
        if first is None:
            first = res
        times = []
        t0 = time.perf_counter()
        while True:
            t1 = time.perf_counter()
            run(threads)
            times.append(time.perf_counter() - t1)
            if time.perf_counter() - t0 >= min_seconds:
                break
        work = amount(threads) if callable(amount) else amount
        rates = [work / t for t in times]
        figures.append({"cores": threads,
                        "value": round(work * len(times) / sum(times), digits),
                        "min": round(min(rates), digits), "max": round(max(rates), digits),
                        "runs": len(times), "seconds": round(sum(times), 2)})
    torch.set_num_threads(all_threads)
    return figures, first


def cpu_baseline(w, min_seconds, sample=None):
    """Time the CPU oracle over `w` on all host threads, then on one thread; GB/s over the
    reference algorithm's bytes.  Returns the cpu_baseline object (all threads, with the
    one-thread figure and the run-to-run spread of both) and the oracle's result for w."""
    from mvsd.testing import configs

    run = cpu_oracle_runner(w)
    nbytes = configs.algorithmic_bytes(w)
    figures, ref = time_on_threads(lambda threads: run(), min_seconds, nbytes / 1e9)
    main = figures[0]
    what = sample or (f"the whole workload ({w.batch_size} requests, {w.num_tokens} verify "
                      f"rows, V={w.vocab_size})")
    return {"value": main["value"], "unit": "GB/s", "cores": main["cores"], "kind": "port",
            "sample": f"{what} through oracle/rejection.py on torch-CPU (the reference "
                      f"algorithm: every row scored"
                      + ("; top-k / top-p by sorting each row" if is_constrained(w) else "")
                      + f"), repeated back to back after one warm-up, on {main['cores']} "
                      f"threads and on 1; GB/s over the reference algorithm's bytes of the "
                      f"sample; min/max are the per-run spread; inputs in host memory, same "
                      f"uniforms and noise as the GPU run",
            "by_cores": figures}, ref


def kernel_sources_sha256(sources):
    import hashlib

    h = hashlib.sha256()
    for rel in sources:
        h.update((ROOT / rel).read_bytes())
    return h.hexdigest()


def load_traffic(config):
    """HBM bytes per call from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary of
    `config` (a line ``traffic_bytes_per_launch[<config>] = N``), used only when the
    summary's ``kernel_sources_sha256`` matches the current sources of that config's
    kernels; else None."""
    if config not in TRAFFIC:
        return None
    path, sources = TRAFFIC[config]
    if not path.exists():
        return None
    value, sha = None, None
    key = f"traffic_bytes_per_launch[{config}] = "
    for line in path.read_text().splitlines():
        if line.startswith(key):
            value = int(line[len(key):].strip())
        if line.startswith("kernel_sources_sha256 = "):
            sha = line.split("=", 1)[1].strip()
    if value is None or sha != kernel_sources_sha256(sources):
        return None
    return value


def parity_summary(w, out, ref):
    """Token parity of the GPU output against the oracle's on the same inputs: requests whose
    output differs, and how many of those differ only at an acceptance margin below 1e-6 or a
    recovered-token near-tie (the allowances of the parity bar); anything else is
    `unexplained` and fails the tests."""
    from oracle import rejection as orc

    rep = orc.compare(out[:w.batch_size].cpu().numpy(), ref, w.draft_token_ids.cpu(),
                      w.num_draft_tokens)
    return {"requests": rep.requests, "mismatched": rep.mismatched,
            "accept_flips": rep.accept_flips, "recovered_flips": rep.recovered_flips,
            "unexplained": len(rep.unexplained)}


def verify_figures(w, ms, wall_ms, out):
    """Byte counts, rates, fractions of peak and accept statistics of one timed verify
    configuration."""
    from mvsd.sample.rejection_sampler import RejectionSampler
    from mvsd.testing import configs

    outputs, _ = RejectionSampler.parse_output(out, w.vocab_size)
    # With top-k / top-p each constrained row must be read once more, by whatever computes its
    # thresholds before the verification (the constraints kernel reads top-p rows three times
    # and top-k rows once; only one pass is counted).
    nbytes = configs.kernel_bytes(w, outputs, constrained_passes=1 if is_constrained(w) else 0)
    ref_bytes = configs.algorithmic_bytes(w)
    tokens = sum(len(o) for o in outputs)
    gbs = nbytes / (ms / 1e3) / 1e9
    ref_gbs = ref_bytes / (ms / 1e3) / 1e9
    return {
        "ms_per_step": round(ms, 5), "wall_ms_per_step": round(wall_ms, 5),
        "kernel_bytes": nbytes, "GBps_on_kernel_bytes": round(gbs, 2),
        "frac_on_kernel_bytes": round(gbs / HBM_PEAK_GBS, 4),
        "reference_algorithm_bytes": ref_bytes, "GBps_on_reference_bytes": round(ref_gbs, 2),
        "frac_on_reference_bytes": round(ref_gbs / HBM_PEAK_GBS, 4),
        "verified_tok_per_s": round(tokens / (ms / 1e3), 1),
        "verified_tokens_per_step": tokens,
        "accept_length_hist": accept_histogram(outputs, w.num_draft_tokens, w.max_spec_len),
        "accept_rate_by_position": accept_rates(outputs, w.num_draft_tokens, w.max_spec_len),
    }


def bench_forward(w, steps, warmup):
    """ms per RejectionSampler.forward call (the drop-in's whole step) on the same rows in the
    compact [P + B, V] layout (k verify rows, then the bonus row, per request): bonus rows
    through mvsd.sample.Sampler, the uniforms and the [B, V] Exp(1) noise drawn by torch's
    generator, then the verification.  Workloads whose target is already compact (C5) use it
    as it is; the headline's verify rows are laid out with a copy of row b as the bonus row
    of request b."""
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
    if w.target_rows is not None:
        assert torch.equal(meta.target_logits_indices.to(torch.int64), w.target_rows.long())
        logits = w.target_logits
    else:
        logits = torch.empty((P + B, V), dtype=w.target_logits.dtype, device=device)
        logits[meta.target_logits_indices.long()] = w.target_logits
        logits[meta.bonus_logits_indices.long()] = w.target_logits[:B]
    temps = w.temperature.tolist()
    sm = sampling_metadata(temps, drafts, device=device)
    rs = RejectionSampler(Sampler())

    def step():
        return rs(meta, w.draft_probs, logits, sm).sampled_token_ids

    ms, wall_ms, _ = time_steps(step, steps, warmup)
    del logits
    dt = "fp32" if w.target_logits.dtype == torch.float32 else "bf16"
    return {"ms_per_step": round(ms, 5), "wall_ms_per_step": round(wall_ms, 5),
            "path": f"RejectionSampler(Sampler()).forward on compact [P + B, V] {dt} logits: "
                    "bonus-row sampling, uniforms and Exp(1) noise from torch's generator, "
                    "verification (no penalties, no logprobs)"}


def bench_verify_config(name, device, steps, warmup, cpu_seconds, with_cpu):
    """One verify configuration (c1, c2, c4, c5) measured as the headline is: the entry of the
    'configs' object."""
    w = make_workload(name, device)
    ms, wall_ms, out = time_steps(run_step(w), steps, warmup)
    entry = {"workload": WORKLOAD_NAMES[name], "steps": steps, "warmup": warmup,
             "dtype": "f32" if w.target_logits.dtype == torch.float32 else "bf16",
             **verify_figures(w, ms, wall_ms, out)}
    traffic = load_traffic(name)
    entry["traffic"] = traffic
    entry["traffic_over_kernel_bytes"] = (None if traffic is None
                                          else round(traffic / entry["kernel_bytes"], 4))
    if name == "c5":
        entry["drop_in_forward"] = bench_forward(w, steps, warmup)
    entry["cpu_baseline"] = entry["parity"] = None
    if with_cpu:
        n = CPU_SAMPLE[name]
        cw = head(w, n)
        entry["cpu_baseline"], ref = cpu_baseline(
            cw, cpu_seconds, None if n is None else
            f"the first {n} of {w.batch_size} requests ({cw.num_tokens} verify rows, "
            f"V={w.vocab_size})")
        pn = PARITY_SAMPLE[name]
        if pn != n:
            pw = head(w, pn)
            ref = cpu_oracle_runner(pw)()
        else:
            pw = cw
        entry["parity"] = parity_summary(pw, out, ref)
        if pn is not None:
            entry["parity"]["sample"] = f"the first {pn} of {w.batch_size} requests"
    del w, out
    torch.cuda.empty_cache()
    return entry


def bench_ngram(device, steps, warmup, with_cpu, cpu_seconds, pmc=False):
    """C3: the ngram proposer over 256 histories of 4096 tokens (``ngram_propose_device``: the
    kernel on device-resident histories), the host-buffer API, and the CPU KMP matcher (the
    reference CPU algorithm) on all host threads (requests split across threads) and on one.
    pmc: run the counter-calibration copy and three steps only."""
    from mvsd.spec_decode.ngram_proposer_gpu import ngram_propose_device
    from mvsd.testing import configs
    from oracle import ngram as ong

    tokens = configs.ngram_c3(device)
    B, L = tokens.shape
    lens = torch.full((B,), L, dtype=torch.int32, device=device)

    def step():
        return ngram_propose_device(tokens, lens, min_n=2, max_n=5, k=5)

    if pmc:
        pmc_driver(step, device)
        return None
    ms, wall_ms, (d, v) = time_steps(step, steps, warmup)
    nbytes = B * L * 4 + B * 4 + B * 5 * 4 + B * 4
    gbs = nbytes / (ms / 1e3) / 1e9
    tn, ln = tokens.cpu().numpy(), lens.cpu().numpy()
    entry = {"workload": "c3 ngram B=256 L=4096 min_n=2 max_n=5 k=5 (int32 histories)",
             "steps": steps, "warmup": warmup, "dtype": "int32",
             "ms_per_step": round(ms, 5), "wall_ms_per_step": round(wall_ms, 5),
             "requests_per_s": round(B / (ms / 1e3), 1), "kernel_bytes": nbytes,
             "GBps_on_kernel_bytes": round(gbs, 2),
             "frac_on_kernel_bytes": round(gbs / HBM_PEAK_GBS, 5),
             "bound": "latency (one 16 KB history per workgroup, 4.2 MB per call; the "
                      "kernel takes about 7 us, the host wrapper and launch the rest)",
             "host_api": None, "cpu_baseline": None, "parity": None}
    traffic = load_traffic("c3")
    entry["traffic"] = traffic
    entry["traffic_over_kernel_bytes"] = None if traffic is None else round(traffic / nbytes, 4)
    host_ms = bench_ngram_host_api(tn, ln, steps, warmup, device)
    entry["host_api"] = {"ms_per_call": round(host_ms, 5),
                         "requests_per_s": round(B / (host_ms / 1e3), 1),
                         "path": "NgramProposer.propose on pageable numpy histories [256, 4096] "
                                 "int32: pinned staging, one upload, the kernel, drafts and "
                                 "counts back, one synchronisation (wall clock)"}
    if with_cpu:
        from concurrent.futures import ThreadPoolExecutor

        pool = ThreadPoolExecutor(max_workers=all_host_threads())

        def run(threads):
            # one whole batch per thread (a batch takes about a millisecond, too short to split);
            # ctypes releases the GIL around the C matcher, so the threads run in parallel
            res = list(pool.map(lambda _: ong.kmp_batch(tn, ln, 2, 5, 8192, 5), range(threads)))
            return res[0]

        figures, (ed, ev) = time_on_threads(run, cpu_seconds, lambda threads: B * threads,
                                            digits=1)
        pool.shutdown()
        main = figures[0]
        entry["cpu_baseline"] = {"value": main["value"], "unit": "requests/s",
                                 "cores": main["cores"], "kind": "port",
                                 "sample": "all 256 histories through oracle/ngram.c KMP (the "
                                           "reference CPU matcher), one whole batch per host "
                                           "thread at a time, repeated back to back after one "
                                           f"warm-up, on {main['cores']} threads and on 1",
                                 "by_cores": figures}
        got_d, got_v = d.cpu().numpy(), v.cpu().numpy()
        # the device proposer's drafts are those of the CPU matcher; rows without a match
        # propose nothing
        same = [(int(ev[b]) == int(got_v[b]))
                and np.array_equal(ed[b, :ev[b]], got_d[b, :got_v[b]]) for b in range(B)]
        entry["parity"] = {"requests": B, "mismatched": int(B - sum(same)),
                           "with_drafts": int((got_v > 0).sum())}
    # the same histories with every other one ending in a copied span: those requests match
    tokens2 = configs.ngram_c3(device, suffix_copies=True)
    ms2, wall2, (d2, v2) = time_steps(
        lambda: ngram_propose_device(tokens2, lens, min_n=2, max_n=5, k=5), steps, warmup)
    sub = {"ms_per_step": round(ms2, 5), "requests_per_s": round(B / (ms2 / 1e3), 1),
           "rows_with_drafts": int((v2 > 0).sum()),
           "histories": "C3's histories, every other one ending with a copy of an earlier span "
                        "of 8-64 tokens (configs.ngram_c3(suffix_copies=True))"}
    if with_cpu:
        kd, kc = ong.kmp_batch(tokens2.cpu().numpy(), ln, 2, 5, 8192, 5)
        g2, c2 = d2.cpu().numpy(), v2.cpu().numpy()
        sub["parity"] = {"requests": B, "mismatched": int(sum(
            1 for b in range(B) if int(kc[b]) != int(c2[b])
            or not np.array_equal(kd[b, :kc[b]], g2[b, :c2[b]])))}
    entry["suffix_copies"] = sub
    return entry


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


def bench_v2(device, steps, warmup, with_cpu, cpu_seconds, pmc=False):
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

    if pmc:
        pmc_driver(step, device)
        return None
    ms, wall_ms, (s, n) = time_steps(step, steps, warmup)
    n_host = n.cpu().numpy()
    s_host = s.cpu().numpy()
    n_bonus = int((n_host == K + 1).sum())
    P = B * K
    nbytes = 2 * P * V * 4 + n_bonus * V * 4 + rows * (4 + 8 + 4 + 4) + B * (4 + 4 + 4 + 8) \
        + B * (K + 1) * 8 + B * 4
    gbs = nbytes / (ms / 1e3) / 1e9
    traffic = load_traffic("v2")
    entry = {"workload": "v2 B=256 k=4 V=151936 fp32 random T=0.8, draft logits [B, k, V]",
             "steps": steps, "warmup": warmup, "dtype": "f32",
             "ms_per_step": round(ms, 5), "wall_ms_per_step": round(wall_ms, 5),
             "kernel_bytes": nbytes, "GBps_on_kernel_bytes": round(gbs, 2),
             "frac_on_kernel_bytes": round(gbs / HBM_PEAK_GBS, 4),
             "kernels": "v2_stats + v2_chain + v2_resample + v2_insert per call",
             "traffic": traffic,
             "traffic_over_kernel_bytes": None if traffic is None else round(traffic / nbytes, 4),
             "verified_tok_per_s": round(float(n_host.sum()) / (ms / 1e3), 1),
             "accept_length_hist": np.bincount(n_host - 1, minlength=K + 1).tolist(),
             "cpu_baseline": None, "parity": None}
    if with_cpu:
        sub = 16  # requests in the CPU sample
        host = {k: (v.cpu().numpy() if isinstance(v, torch.Tensor) else v)
                for k, v in case.items()}
        r_rows = sub * (K + 1)
        host["target_logits"] = host["target_logits"][:r_rows]
        for k in ("draft_sampled", "pos", "expanded_idx_mapping", "expanded_local_pos"):
            host[k] = host[k][:r_rows]
        host["cu_num_logits"] = host["cu_num_logits"][:sub + 1]
        host["idx_mapping"] = host["idx_mapping"][:sub]
        sub_bytes = nbytes * sub / B
        figures, res = time_on_threads(
            lambda threads: ov2.rejection_sample(**host, return_margins=True,
                                                 return_windows=True),
            cpu_seconds, sub_bytes / 1e9)
        es, en, margins, gaps, wins, gap_wins = res
        main = figures[0]
        entry["cpu_baseline"] = {"value": main["value"], "unit": "GB/s", "cores": main["cores"],
                                 "kind": "port",
                                 "sample": f"the first {sub} of {B} requests through "
                                           "oracle/v2_rejection.py (numpy), repeated back to back "
                                           "after one warm-up, on all host threads and on 1 "
                                           "(numpy's reductions are single-threaded)",
                                 "by_cores": figures}
        same = [int(n_host[r]) == int(en[r]) and np.array_equal(s_host[r, :en[r]], es[r, :en[r]])
                for r in range(sub)]
        near = [any(m < w for m, w in zip(margins[r], wins[r])) or gaps[r] < gap_wins[r]
                for r in range(sub)]
        entry["parity"] = {"requests": sub, "mismatched": int(sub - sum(same)),
                           "near_tie_flips": int(sum(1 for a, b in zip(same, near)
                                                     if not a and b)),
                           "unexplained": int(sum(1 for a, b in zip(same, near)
                                                  if not a and not b)),
                           "decisions_inside_flip_window": int(sum(near)),
                           "sample": f"the first {sub} of {B} requests"}
    del case, target, draft
    torch.cuda.empty_cache()
    return entry


def pmc_driver(step, device):
    """The counter-calibration copy (reads 1 GiB, writes 1 GiB) and three steps."""
    a = torch.empty(256 * 1024 * 1024, dtype=torch.float32, device=device)  # 1 GiB
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    del a, b
    for _ in range(3):
        step()
    torch.cuda.synchronize()


def verify_line(name, args, device):
    """The JSON line of one verify configuration (the headline by default)."""
    w = make_workload(name, device)
    step = run_step(w)
    if args.pmc_driver:
        pmc_driver(step, device)
        return None
    ms, wall_ms, out = time_steps(step, args.steps, args.warmup)
    fig = verify_figures(w, ms, wall_ms, out)
    gbs = fig["GBps_on_kernel_bytes"]
    constrained = is_constrained(w)
    line = {
        "metric": METRIC,
        "value": gbs,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": fig["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if w.target_logits.dtype == torch.float32 else "bf16",
        "data": "synthetic (seeded on-device Philox; random logits, no checkpoint)",
        "config": {"workload": WORKLOAD_NAMES[name],
                   "batch_size": w.batch_size, "num_draft_rows": w.num_tokens,
                   "vocab_size": w.vocab_size,
                   "kernel_bytes": fig["kernel_bytes"],
                   "reference_algorithm_bytes": fig["reference_algorithm_bytes"],
                   "effective_GBps_on_reference_bytes": fig["GBps_on_reference_bytes"]},
        "pct_of_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "verified_tok_per_s": fig["verified_tok_per_s"],
        "verified_tokens_per_step": fig["verified_tokens_per_step"],
        "accept_length_hist": fig["accept_length_hist"],
        "accept_rate_by_position": fig["accept_rate_by_position"],
        "wall_ms_per_step": fig["wall_ms_per_step"],
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": load_traffic(name),
                     "kernel": ("mvsd::verify_kernel"
                                + (" + plan + constraints_kernel" if constrained else "")
                                + " per rejection_sample"),
                     "kernel_ms": fig["ms_per_step"],
                     "clock": "the timed region: HIP events on the launch stream around the "
                              "steps back to back, divided by the step count (the verify "
                              "kernel is the step's only launch)"},
        "cpu_baseline": None,
        "parity": None,
    }
    if name in ("h", "c5"):
        line["drop_in_forward"] = bench_forward(w, args.steps, args.warmup)
    if not args.no_cpu_baseline:
        n = CPU_SAMPLE[name]
        cw = head(w, n)
        line["cpu_baseline"], ref = cpu_baseline(
            cw, args.cpu_seconds, None if n is None else
            f"the first {n} of {w.batch_size} requests ({cw.num_tokens} verify rows)")
        line["parity"] = parity_summary(cw, out, ref)
    del w, out
    torch.cuda.empty_cache()
    return line


def main():
    args = parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 "
                          "(request or vocabulary sharding across GPUs is not launched)"}))
        sys.exit(2)
    device = torch.device("cuda", 0)
    with_cpu = not args.no_cpu_baseline
    if args.config == "c3" and args.pmc_driver:
        bench_ngram(device, args.steps, args.warmup, False, 0.0, pmc=True)
        return
    if args.config == "c3":
        line = {"metric": "ngram proposer drafts/s (C3)", "n_gpus": 1, "unit": "requests/s",
                "higher_is_better": True, "scaling": "strong", "vs_baseline": None,
                "data": "synthetic (seeded numpy histories with copied spans)",
                "config": {"workload": "c3 ngram B=256 L=4096 min_n=2 max_n=5 k=5"},
                **bench_ngram(device, args.steps, args.warmup, with_cpu, args.cpu_seconds)}
        line["value"] = line["requests_per_s"]
        print(json.dumps(line), flush=True)
        return
    if args.config == "v2" and args.pmc_driver:
        bench_v2(device, args.steps, args.warmup, False, 0.0, pmc=True)
        return
    if args.config == "v2":
        line = {"metric": "V2 rejection-sampler HBM GB/s (% of peak) + verified tok/s, "
                          "B=256 k=4 V=152k", "n_gpus": 1, "unit": "GB/s",
                "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
                "data": "synthetic (seeded torch generator on device; no checkpoint)",
                "config": {"workload": "v2 B=256 k=4 V=151936 fp32 random T=0.8"},
                **bench_v2(device, args.steps, args.warmup, with_cpu, args.cpu_seconds)}
        line["value"] = line["GBps_on_kernel_bytes"]
        print(json.dumps(line), flush=True)
        return
    line = verify_line(args.config, args, device)
    if line is None:
        return
    if args.config == "h" and args.configs != "none":
        line["configs"] = {}
        for name in [c for c in args.configs.split(",") if c]:
            print(f"[bench] {name}", file=sys.stderr, flush=True)
            if name == "c3":
                entry = bench_ngram(device, args.sub_steps, args.warmup, with_cpu,
                                    args.sub_cpu_seconds)
            elif name == "v2":
                entry = bench_v2(device, args.sub_steps, args.warmup, with_cpu,
                                 args.sub_cpu_seconds)
            else:
                entry = bench_verify_config(name, device, args.sub_steps, args.warmup,
                                            args.sub_cpu_seconds, with_cpu)
            line["configs"][name] = entry
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
