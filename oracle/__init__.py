"""TEST INFRASTRUCTURE ONLY: CPU restatement of the reference rules (the checker)."""
