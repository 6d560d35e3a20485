"""Test-only CPU oracle for First Passage Attention (see fpa_oracle.py's header)."""
