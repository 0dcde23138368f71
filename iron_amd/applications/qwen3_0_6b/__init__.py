"""Qwen3 int8 decode runtime."""
