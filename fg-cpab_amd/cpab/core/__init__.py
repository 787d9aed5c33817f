"""Host-side tessellation and basis construction for CPAB transformations."""
