"""Compressed-tensors INT4/INT8 checkpoints behind a pluggable fused Linear."""
