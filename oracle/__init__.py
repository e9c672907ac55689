"""CPU oracle of the INT8 KV-cache hot path (test infrastructure; see int8kv_oracle)."""
