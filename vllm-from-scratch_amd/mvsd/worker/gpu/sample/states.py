"""Constants of the V2 sampling states (minivllm/worker/gpu/sample/states.py:30)."""

# A request that asked for no logprobs (max_num_logprobs of a batch without any).
NO_LOGPROBS = -1
