"""Utilities: phase ranges for profilers (``signpost``)."""
