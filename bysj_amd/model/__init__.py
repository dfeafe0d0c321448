"""DeepMD seam binder and ``DPA4Model`` facade (the reference's ``model`` package)."""

from .dpa4 import DPA4Model

__all__ = ["DPA4Model"]
