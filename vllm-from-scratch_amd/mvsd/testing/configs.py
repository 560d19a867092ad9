"""Synthetic verification workloads (the benchmark configurations), generated on the device.

Every tensor comes from a seeded ``torch.Generator`` on the target device (Philox4x32-10 on
ROCm), seed ``1000 + config number``; the same tensors are handed to the HIP path and, copied
to the host, to the CPU oracle, so both see identical inputs, uniforms and noise.

    c1  greedy,  B=4,    k=3, V=151936, fp32 logits N(0, 2^2); half the drafts set to the
        row argmax; bonus = argmax of each request's bonus row
    c2  random,  B=64,   k=4, fp32; draft logits D ~ N(0, 2^2), target = D + N(0, 0.5^2),
        T=0.8, draft_probs = softmax(D / T), drafts sampled from draft_probs
    h   headline: c2's recipe at B=256, k=4 (P=1024)
    c4  ragged mixed: B=512, K_i ~ U{0..8}, half greedy / half random T ~ U[0.3, 1.5],
        bf16 logits correlated as in c2 (top-k / top-p quartiles are attached as metadata)
    c5  EAGLE-style: B=1024, k=7, bf16 target [B*8, V] ~ N(0, 2.5^2), draft_probs =
        softmax(target + N(0, 1)) at T=1, full recovered + bonus path
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

VOCAB = 151936


@dataclass
class Workload:
    name: str
    num_draft_tokens: list[int]
    max_spec_len: int
    draft_token_ids: torch.Tensor          # [P] int32
    cu_num_draft_tokens: torch.Tensor      # [B] int32
    target_logits: torch.Tensor            # [P, V] (or [P+B, V] with target_rows)
    target_rows: torch.Tensor | None       # [P] int32 rows into target_logits, or None
    draft_probs: torch.Tensor | None       # [P, V] fp32
    bonus_token_ids: torch.Tensor          # [B, 1] int32
    temperature: torch.Tensor | None       # [B] fp32 (None = all greedy)
    all_greedy: bool
    all_random: bool
    uniforms: torch.Tensor | None          # [P] fp64
    exp_noise: torch.Tensor | None         # [B, V] fp32
    apply_temperature: bool = True         # temperature applied in the kernel
    top_k: torch.Tensor | None = None      # [B] int64 (V = off)
    top_p: torch.Tensor | None = None      # [B] fp32 (1.0 = off)
    extra: dict = field(default_factory=dict)

    @property
    def batch_size(self) -> int:
        return len(self.num_draft_tokens)

    @property
    def num_tokens(self) -> int:
        return int(self.draft_token_ids.shape[0])

    @property
    def vocab_size(self) -> int:
        return int(self.target_logits.shape[-1])


def _gen(device, seed):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _cu(ks: list[int], device) -> torch.Tensor:
    return torch.tensor(np.cumsum(ks), dtype=torch.int32, device=device)


def _exp_noise(B, V, g, device):
    e = torch.empty((B, V), dtype=torch.float32, device=device).exponential_(generator=g)
    return e.clamp_min_(torch.finfo(torch.float32).tiny)


def _uniforms(P, g, device):
    u = torch.rand((P,), dtype=torch.float64, device=device, generator=g)
    return u.clamp_min_(1e-300)


def _sample_from(probs: torch.Tensor, g) -> torch.Tensor:
    """Exponential race per row (harness-side draft sampling)."""
    e = torch.empty_like(probs).exponential_(generator=g)
    return (probs / e).argmax(dim=-1).to(torch.int32)


def greedy_c1(device, B=4, k=3, V=VOCAB, seed=1001) -> Workload:
    g = _gen(device, seed)
    ks = [k] * B
    # compact rows: k verify rows then the bonus row, per request
    logits = torch.randn((B * (k + 1), V), device=device, generator=g) * 2.0
    rows = torch.arange(B * (k + 1), device=device).view(B, k + 1)
    target_rows = rows[:, :k].reshape(-1).to(torch.int32)
    bonus_rows = rows[:, k]
    argmax = logits.argmax(dim=-1)
    drafts = torch.randint(0, V, (B * k,), device=device, generator=g)
    take = torch.rand((B * k,), device=device, generator=g) < 0.5
    drafts = torch.where(take, argmax[target_rows.long()], drafts).to(torch.int32)
    bonus = argmax[bonus_rows].to(torch.int32).view(B, 1)
    return Workload("c1", ks, k, drafts, _cu(ks, device), logits, target_rows, None, bonus,
                    None, True, False, None, None)


def random_c2(device, B=64, k=4, V=VOCAB, T=0.8, seed=1002, name="c2") -> Workload:
    g = _gen(device, seed)
    ks = [k] * B
    P = B * k
    draft_logits = torch.randn((P, V), device=device, generator=g) * 2.0
    target = draft_logits + torch.randn((P, V), device=device, generator=g) * 0.5
    draft_probs = torch.softmax(draft_logits / T, dim=-1)
    del draft_logits
    drafts = _sample_from(draft_probs, g)
    bonus = torch.randint(0, V, (B, 1), device=device, generator=g, dtype=torch.int32)
    temperature = torch.full((B,), T, dtype=torch.float32, device=device)
    return Workload(name, ks, k, drafts, _cu(ks, device), target, None, draft_probs, bonus,
                    temperature, False, True, _uniforms(P, g, device),
                    _exp_noise(B, V, g, device))


def headline(device, B=256, k=4, V=VOCAB) -> Workload:
    return random_c2(device, B=B, k=k, V=V, seed=1000, name="h")


def ragged_c4(device, B=512, V=VOCAB, seed=1004, max_k=8) -> Workload:
    g = _gen(device, seed)
    gen_cpu = torch.Generator().manual_seed(seed)
    ks = torch.randint(0, max_k + 1, (B,), generator=gen_cpu).tolist()
    P = int(sum(ks))
    greedy = torch.zeros(B, dtype=torch.bool)
    greedy[torch.randperm(B, generator=gen_cpu)[: B // 2]] = True
    temps = torch.empty(B).uniform_(0.3, 1.5, generator=gen_cpu)
    temps[greedy] = 0.0
    perm = torch.randperm(B, generator=gen_cpu)
    top_k = torch.full((B,), V, dtype=torch.int64)
    top_p = torch.ones(B, dtype=torch.float32)
    top_k[perm[: B // 4]] = 50
    top_p[perm[B // 4: B // 2]] = 0.9
    draft_bf16 = (torch.randn((P, V), device=device, generator=g) * 2.0).to(torch.bfloat16)
    target_bf16 = (draft_bf16.float() + torch.randn((P, V), device=device, generator=g) * 0.5
                   ).to(torch.bfloat16)
    req = torch.repeat_interleave(torch.arange(B), torch.tensor(ks))
    row_t = temps[req].to(device)
    row_t = torch.where(row_t == 0, torch.ones_like(row_t), row_t)
    draft_probs = torch.softmax(draft_bf16.float() / row_t.unsqueeze(-1), dim=-1)
    drafts = _sample_from(draft_probs, g)
    bonus = torch.randint(0, V, (B, 1), device=device, generator=g, dtype=torch.int32)
    return Workload("c4", ks, max(ks), drafts, _cu(ks, device), target_bf16, None, draft_probs,
                    bonus, temps.to(device), False, False, _uniforms(P, g, device),
                    _exp_noise(B, V, g, device), top_k=top_k.to(device),
                    top_p=top_p.to(device), extra={"draft_logits": draft_bf16})


def eagle_c5(device, B=1024, k=7, V=VOCAB, seed=1005) -> Workload:
    g = _gen(device, seed)
    ks = [k] * B
    P = B * k
    target = (torch.randn((B * (k + 1), V), device=device, generator=g) * 2.5).to(torch.bfloat16)
    rows = torch.arange(B * (k + 1), device=device).view(B, k + 1)
    target_rows = rows[:, :k].reshape(-1).to(torch.int32)
    draft_probs = torch.empty((P, V), dtype=torch.float32, device=device)
    for s in range(0, P, 1024):  # bounded temporaries
        e = min(P, s + 1024)
        x = target[target_rows[s:e].long()].float()
        x += torch.randn(x.shape, device=device, generator=g)
        draft_probs[s:e] = torch.softmax(x, dim=-1)
        del x
    drafts = torch.empty((P,), dtype=torch.int32, device=device)
    for s in range(0, P, 1024):
        e = min(P, s + 1024)
        drafts[s:e] = _sample_from(draft_probs[s:e], g)
    bonus = torch.randint(0, V, (B, 1), device=device, generator=g, dtype=torch.int32)
    temperature = torch.ones((B,), dtype=torch.float32, device=device)
    return Workload("c5", ks, k, drafts, _cu(ks, device), target, target_rows, draft_probs,
                    bonus, temperature, False, True, _uniforms(P, g, device),
                    _exp_noise(B, V, g, device))


def ngram_c3(device, B=256, L=4096, V=VOCAB, seed=1003, copy_frac=0.3, suffix_copies=False):
    """Histories [B, L] int32 uniform in [0, V) with ~copy_frac of each overwritten by copies
    of earlier spans of length 8..64 at random offsets (generated on the host).  A copy never
    covers a history's last token, so no suffix repeats and no request finds a match.  With
    ``suffix_copies`` every other history (even rows) then ends with a copy of an earlier span
    of 8..64 tokens, so those requests match at max_n (prompt lookup's useful case)."""
    rng = np.random.default_rng(seed)
    tokens = rng.integers(0, V, size=(B, L), dtype=np.int64).astype(np.int32)
    for b in range(B):
        written = 0
        while written < copy_frac * L:
            n = int(rng.integers(8, 65))
            dst = int(rng.integers(n, L - n))
            src = int(rng.integers(0, dst - n + 1))
            tokens[b, dst:dst + n] = tokens[b, src:src + n]
            written += n
    if suffix_copies:
        tail = np.random.default_rng(seed + 1)
        for b in range(0, B, 2):
            n = int(tail.integers(8, 65))
            src = int(tail.integers(0, L - 2 * n))
            tokens[b, L - n:] = tokens[b, src:src + n]
    return torch.from_numpy(tokens).to(device)


def algorithmic_bytes(w: Workload) -> int:
    """Bytes the reference algorithm must read once plus the output written once:
    target rows, draft rows of random requests, noise rows of random requests with drafts,
    uniforms/draft ids/cu/bonus/temperature, output."""
    V = w.vocab_size
    ks = np.asarray(w.num_draft_tokens)
    if w.all_greedy:
        greedy = np.ones(len(ks), dtype=bool)
    else:
        greedy = (w.temperature.cpu().numpy() == 0.0)
    P = int(ks.sum())
    P_random = int(ks[~greedy].sum())
    B_random = int(((ks > 0) & ~greedy).sum())
    t_size = w.target_logits.element_size()
    total = P * V * t_size
    if w.draft_probs is not None:
        total += P_random * V * w.draft_probs.element_size()
    total += B_random * V * 4
    total += P * 8 + P * 4 + 4 * len(ks) * 4
    total += len(ks) * (w.max_spec_len + 1) * 4
    return int(total)


def kernel_bytes(w: Workload, outputs: list[list[int]], *, draft_none: bool = False,
                 constrained_passes: int = 0) -> int:
    """Bytes the verify kernel's algorithm must move for workload w, given the run's own output
    (``parse_output`` lists): every verify row of the target once (softmax statistics or greedy
    argmax); for each random request that rejects a draft, that one row's target, draft and
    noise row once more (the recovered-token scores of the first rejected row, the only ones
    the output uses); the per-row decision inputs (draft id, uniform, q[d], x[d]); the
    per-request metadata; the output.  With sampling constraints, each constrained verify row
    is read `constrained_passes` more times by the constraints kernel and its 16-byte row mask
    is written and read."""
    V = w.vocab_size
    ks = np.asarray(w.num_draft_tokens)
    if w.all_greedy:
        greedy = np.ones(len(ks), dtype=bool)
    else:
        greedy = (w.temperature.cpu().numpy() == 0.0)
    P = int(ks.sum())
    t_size = w.target_logits.element_size()
    d_size = 0 if (draft_none or w.draft_probs is None) else w.draft_probs.element_size()
    rejected = sum(1 for r, out in enumerate(outputs)
                   if ks[r] > 0 and not greedy[r] and len(out) <= ks[r])
    total = P * V * t_size
    total += rejected * V * (t_size + d_size + 4)
    total += P * (4 + 8 + d_size + t_size)
    total += len(ks) * 4 * 4
    total += len(ks) * (w.max_spec_len + 1) * 4
    if constrained_passes and (w.top_k is not None or w.top_p is not None):
        on = np.zeros(len(ks), dtype=bool)
        if w.top_k is not None:
            on |= w.top_k.cpu().numpy() < V
        if w.top_p is not None:
            on |= w.top_p.cpu().numpy() < 1.0
        # greedy rows of a batch with random requests are masked too (rejection_sampler.py:549-571)
        rows = 0 if w.all_greedy else int(ks[on].sum())
        total += rows * V * t_size * constrained_passes + P * 16 * 2
    return int(total)
