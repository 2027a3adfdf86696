"""Measurement probes for bench.py (not part of the MSDA library or its boundary)."""
