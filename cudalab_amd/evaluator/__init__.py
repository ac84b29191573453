"""Operator-agnostic evaluation plumbing used by the GEMV path: correctness
metrics, the negative-case runner, the timing pool and GPU snapshots."""
