"""Approximation backends for physical device equations."""
