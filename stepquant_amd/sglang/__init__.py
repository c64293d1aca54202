"""Serving-adapter side of the pool (reference stepquant/sglang): plan
artifacts, per-layer plans and the mamba-pool lifecycle hooks in ``runtime``."""
