"""Operator package (see op.py)."""
