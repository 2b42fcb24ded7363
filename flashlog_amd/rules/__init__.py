"""Rule-bank scoring on the GPU (the reference's rules/shared_inference.py and
rules/max_inference.py entry points)."""
from . import max_inference, shared_inference  # noqa: F401
