"""Prompt-lookup proposer with the host-buffer API (drop-in for
minivllm/spec_decode/ngram_proposer.py).

Same constructor and methods as the reference (``propose``, ``batch_propose``,
``propose_drafts``, ``load_model``, ``remove_requests``) and the same matching rules
(:41-99): the longest n in [prompt_lookup_min, prompt_lookup_max] whose n-gram suffix
occurred earlier, the earliest such occurrence, ``k = min(k, max_model_len - len)`` and
``min(k, tokens after the match)`` drafts.  The match itself runs on the GPU
(``mvsd_ngram_propose`` with the max_model_len cap enabled).  Per call the histories,
lengths and active flags are written into one pinned host buffer and uploaded in one
asynchronous copy; the drafts and counts come back through pinned buffers with one
synchronisation.
"""

from __future__ import annotations

import numpy as np
import torch

from ..outputs import DraftTokenIds
from .ngram_proposer_gpu import ngram_propose_device
from .utils import TargetRows


class NgramProposer:
    def __init__(self, vllm_config, device: torch.device | str | None = None) -> None:
        spec_config = vllm_config.speculative_config
        assert spec_config is not None
        assert spec_config.prompt_lookup_min is not None
        assert spec_config.prompt_lookup_max is not None
        self.min_n = spec_config.prompt_lookup_min
        self.max_n = spec_config.prompt_lookup_max
        self.k = spec_config.num_speculative_tokens
        self.max_model_len = vllm_config.model_config.max_model_len
        max_num_seqs = vllm_config.scheduler_config.max_num_seqs
        self.valid_ngram_draft = np.zeros((max_num_seqs, self.k), dtype=np.int32)
        self.valid_ngram_num_drafts = np.zeros(max_num_seqs, dtype=np.int32)
        self.device = torch.device(device) if device is not None else None
        # pinned staging (grown on demand): [tokens int32 | lengths int32 | active u8] up, and
        # drafts / counts back; each call ends with a synchronisation, so reuse is safe
        self._up_host: torch.Tensor | None = None
        self._up_dev: torch.Tensor | None = None
        self._down_host: torch.Tensor | None = None

    def _device(self) -> torch.device:
        if self.device is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        return self.device

    def propose(self, num_speculative_tokens: int, sampled_token_ids: list[list[int]],
                num_tokens_no_spec: np.ndarray, token_ids_cpu: np.ndarray,
                slot_mappings=None) -> list[list[int]]:
        """Skip requests that sampled nothing this step or reached max_model_len (:124-150)."""
        assert num_speculative_tokens <= self.k
        valid = [i for i, ids in enumerate(sampled_token_ids)
                 if len(ids) and num_tokens_no_spec[i] < self.max_model_len]
        return self.batch_propose(len(sampled_token_ids), valid, num_tokens_no_spec,
                                  token_ids_cpu, num_speculative_tokens)

    def batch_propose(self, num_requests: int, valid_ngram_requests: list,
                      num_tokens_no_spec: np.ndarray, token_ids_cpu: np.ndarray,
                      k: int) -> list[list[int]]:
        """Drafts for ``valid_ngram_requests``; the others get ``[]`` (:152-184)."""
        valid = [int(i) for i in valid_ngram_requests]
        if valid:
            self.valid_ngram_draft[:] = 0
            self.valid_ngram_num_drafts[:] = 0
        if valid and k > 0:
            lengths = np.asarray(num_tokens_no_spec[:num_requests], dtype=np.int64)
            width = max(1, int(lengths[valid].max()))
            width = min(width, token_ids_cpu.shape[1])
            tokens, lens, act = self._upload(token_ids_cpu, lengths, valid, num_requests, width)
            drafts, counts = ngram_propose_device(
                tokens, lens, min_n=self.min_n, max_n=self.max_n, k=k, active=act,
                cap_by_model_len=True, max_model_len=self.max_model_len)
            drafts_np, counts_np = self._download(drafts, counts)
            for i in valid:
                n = int(counts_np[i])
                self.valid_ngram_num_drafts[i] = n
                if n:
                    self.valid_ngram_draft[i, :n] = drafts_np[i, :n]
        valid_set = set(valid)
        out: list[list[int]] = []
        for i in range(num_requests):
            if i in valid_set and self.valid_ngram_num_drafts[i] > 0:
                out.append(self.valid_ngram_draft[i, :self.valid_ngram_num_drafts[i]].tolist())
            else:
                out.append([])
        return out

    def _upload(self, token_ids_cpu: np.ndarray, lengths: np.ndarray, valid: list[int],
                num_requests: int, width: int):
        """Stage rows [:num_requests, :width], their lengths and the active flags in the
        pinned buffer and copy them to the device at once; returns device views."""
        n_tok = num_requests * width * 4
        n_len = num_requests * 4
        need = n_tok + n_len + num_requests
        device = self._device()
        if self._up_host is None or self._up_host.numel() < need:
            size = max(need, 2 * (0 if self._up_host is None else self._up_host.numel()))
            self._up_host = torch.empty(size, dtype=torch.uint8, pin_memory=True)
            self._up_dev = torch.empty(size, dtype=torch.uint8, device=device)
        host = self._up_host.numpy()
        host[:n_tok].view(np.int32).reshape(num_requests, width)[:] = \
            token_ids_cpu[:num_requests, :width]
        host[n_tok:n_tok + n_len].view(np.int32)[:] = np.minimum(lengths, width)
        flags = host[n_tok + n_len:need]
        flags[:] = 0
        flags[valid] = 1
        dev = self._up_dev
        dev[:need].copy_(self._up_host[:need], non_blocking=True)
        tokens = dev[:n_tok].view(torch.int32).view(num_requests, width)
        return tokens, dev[n_tok:n_tok + n_len].view(torch.int32), dev[n_tok + n_len:need]

    def _download(self, drafts: torch.Tensor, counts: torch.Tensor):
        """Copy drafts [B, k] and counts [B] (int32) back through pinned memory; one sync."""
        B, k = drafts.shape
        need = B * (k + 1)
        if self._down_host is None or self._down_host.numel() < need:
            self._down_host = torch.empty(max(need, 1024), dtype=torch.int32, pin_memory=True)
        host = self._down_host
        host[:B * k].view(B, k).copy_(drafts, non_blocking=True)
        host[B * k:need].copy_(counts, non_blocking=True)
        torch.cuda.current_stream(drafts.device).synchronize()
        out = host.numpy()
        return out[:B * k].reshape(B, k).copy(), out[B * k:need].copy()

    def load_model(self, *args, **kwargs):
        pass

    def propose_drafts(self, rows: list[TargetRows], all_token_ids: dict[str, list[int]],
                       input_batch=None, reset_req_ids: set[str] | None = None,
                       num_speculative_tokens: int | None = None) -> DraftTokenIds:
        """The runner's proposer protocol (:192-238)."""
        if num_speculative_tokens is None:
            num_speculative_tokens = self.k
        if not 0 <= num_speculative_tokens <= self.k:
            raise ValueError(f"K={num_speculative_tokens} is outside [0, {self.k}]")
        if input_batch is not None:
            token_ids = input_batch.token_ids_cpu.numpy()
            num_tokens_no_spec = input_batch.num_tokens_no_spec.numpy()
        else:
            token_ids, num_tokens_no_spec = self._history_table(rows, all_token_ids)
        sampled = [[0] if target.ready else [] for target in rows]
        drafts = self.propose(num_speculative_tokens, sampled, num_tokens_no_spec, token_ids)
        return DraftTokenIds(req_ids=[t.req_id for t in rows], draft_token_ids=drafts)

    def _history_table(self, rows: list[TargetRows], all_token_ids: dict[str, list[int]]):
        """The batch buffers built from token lists: an int32 table [len(rows), max_model_len]
        whose row i starts with request rows[i]'s committed tokens (at most history_end of
        them, cut at max_model_len) and is zero after them, and those lengths."""
        width = self.max_model_len
        kept = [all_token_ids[t.req_id][:t.history_end][:width] for t in rows]
        lengths = np.array([len(h) for h in kept], dtype=np.int32)
        table = np.zeros((len(rows), width), dtype=np.int32)
        if lengths.sum():
            # a boolean mask fills row-major order, which is the order of the concatenation
            table[np.arange(width)[None, :] < lengths[:, None]] = np.concatenate(
                [np.asarray(h, dtype=np.int32) for h in kept if len(h)])
        return table, lengths

    def remove_requests(self, req_ids) -> None:
        pass
