"""CPU oracle of the paged-KV hot path: test infrastructure only (see paged_kv.py)."""
