"""Serving-engine integrations of the FragPack store and kernels."""
