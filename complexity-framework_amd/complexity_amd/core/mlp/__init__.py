"""MLP plug-ins; importing registers ``tr_hash_engine`` / ``tr_hash_moe``."""

from .base import MLPBase, MLPConfig
from .tr_hash_engine import TRHashEngineMLP

__all__ = ["MLPBase", "MLPConfig", "TRHashEngineMLP"]
