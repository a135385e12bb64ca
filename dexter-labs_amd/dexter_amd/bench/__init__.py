"""Workload definitions and timing helpers for the attention path."""
