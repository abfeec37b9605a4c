"""CPU oracle package (test infrastructure only; never imported by spira_amd)."""
