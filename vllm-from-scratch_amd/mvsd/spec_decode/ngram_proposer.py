"""Prompt-lookup proposer with the host-buffer API (drop-in for
minivllm/spec_decode/ngram_proposer.py).

Same constructor and methods as the reference (``propose``, ``batch_propose``,
``propose_drafts``, ``load_model``, ``remove_requests``) and the same matching rules
(:41-99): the longest n in [prompt_lookup_min, prompt_lookup_max] whose n-gram suffix
occurred earlier, the earliest such occurrence, ``k = min(k, max_model_len - len)`` and
``min(k, tokens after the match)`` drafts.  The match itself runs on the GPU
(``mvsd_ngram_propose`` with the max_model_len cap enabled): the valid rows' histories are
uploaded once per call and the ``[B, k]`` drafts come back in one copy.
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
            rows = np.ascontiguousarray(token_ids_cpu[:num_requests, :width], dtype=np.int32)
            active = np.zeros(num_requests, dtype=np.uint8)
            active[valid] = 1
            device = self._device()
            tokens = torch.from_numpy(rows).to(device)
            lens = torch.from_numpy(np.minimum(lengths, width).astype(np.int32)).to(device)
            act = torch.from_numpy(active).to(device)
            drafts, counts = ngram_propose_device(
                tokens, lens, min_n=self.min_n, max_n=self.max_n, k=k, active=act,
                cap_by_model_len=True, max_model_len=self.max_model_len)
            drafts_np = drafts.cpu().numpy()
            counts_np = counts.cpu().numpy()
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
            token_ids = np.zeros((len(rows), self.max_model_len), dtype=np.int32)
            num_tokens_no_spec = np.zeros(len(rows), dtype=np.int32)
            for index, target in enumerate(rows):
                tokens = all_token_ids[target.req_id][:target.history_end]
                length = min(len(tokens), self.max_model_len)
                token_ids[index, :length] = tokens[:length]
                num_tokens_no_spec[index] = length
        sampled = [[0] if target.ready else [] for target in rows]
        drafts = self.propose(num_speculative_tokens, sampled, num_tokens_no_spec, token_ids)
        return DraftTokenIds(req_ids=[t.req_id for t in rows], draft_token_ids=drafts)

    def remove_requests(self, req_ids) -> None:
        pass
