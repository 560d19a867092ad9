"""Mirror of minivllm/worker/gpu: the V2 model runner's speculative-decoding verification."""
