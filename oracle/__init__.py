"""TEST INFRASTRUCTURE ONLY: CPU oracle of the CPAB hot path (see oracle.py)."""
