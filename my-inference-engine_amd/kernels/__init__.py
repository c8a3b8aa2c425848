"""MI355X attention kernels behind the reference engine's `kernels` package interface."""
