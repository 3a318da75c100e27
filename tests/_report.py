"""Parity figures the GPU tests measured in this session (printed at the end of the run)."""
LINES = []
