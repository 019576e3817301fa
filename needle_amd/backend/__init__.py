"""Block-id contract and the continuous-batching driver around the paged-KV path."""
