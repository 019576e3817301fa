"""Model-side pieces the paged-KV path needs: config parsing and the Qwen2/Llama decoder."""
