"""Kernel-facing Python API (mirrors the reference's kernel/ package)."""
