"""re-export of the oracle's host-layer helpers for the tests"""
from hostlayer import HostLayer, x_rows, parity, parity_ulp, bf16_ulp, MAX_ABS, MEAN_REL, H, I, E  # noqa: F401
