"""CPU oracle for Origami's canonical KV codec layout (test infrastructure only)."""
