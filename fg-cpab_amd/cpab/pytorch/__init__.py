"""PyTorch front end of the MI355X CPAB transform (HIP kernels behind a C ABI)."""
