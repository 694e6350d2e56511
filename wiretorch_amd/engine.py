"""Placeholder, replaced by the HIP engine."""


def simulate(*args, **kwargs):
    raise RuntimeError("the HIP engine is not built")
