"""CPU oracle for the codec/vocoder decode path (test infrastructure only)."""
