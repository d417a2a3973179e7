"""nn.Module wrappers with the reference interfaces."""

from .flash_gqa import FastestFlashGQA
from .flash_mha import FastestFlashMHA
from .flash_mla import FastestFlashMLA

__all__ = ["FastestFlashMHA", "FastestFlashGQA", "FastestFlashMLA"]
