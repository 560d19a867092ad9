"""Mirror of minivllm/worker: only the V2 (gpu/) verification path is built here."""
