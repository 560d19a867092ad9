"""Mirror of minivllm/worker/gpu/sample: the pieces the V2 verification path calls."""
