"""CPU oracle of the paged-KV decode path (test infrastructure only; see
paged_oracle.py for who may import it)."""
