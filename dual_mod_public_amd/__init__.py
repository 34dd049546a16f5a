"""MI355X-native Dual-Mod attention hot path (HIP/CDNA4 kernels behind a C-ABI)."""

from .config import DualModConfig  # noqa: F401

__version__ = "0.1.0"
