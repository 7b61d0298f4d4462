"""CPU oracle of nano-vllm's attention hot path (test infrastructure only)."""
