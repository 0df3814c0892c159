"""CPU oracle package (test infrastructure only; see attention_ref.py)."""
