"""CPU oracle for the paged KV-cache path (test infrastructure only)."""
