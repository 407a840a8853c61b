"""Test-only CPU oracle for the MI355X VSA hot path (see vsa_oracle.py)."""
