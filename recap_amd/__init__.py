"""MI355X-native RECAP corrected sparse attention.

The operator surface of lyraxtg/RECAP (``Operator``, ``HostBankOperator``, the config
loader and the EXACT / REFRESH / SPARSE call kinds) over hand-written gfx950 HIP kernels
behind the C ABI of ``librecap_hip.so`` (include/recap_hip.h).
"""

from .config import (OperatingPoint, OperatorConfig, RecapConfig, config_from_dict,
                     load_config)
from .layout import Layout, SparseGeometry, hilbert_permutation
from .operator import EXACT, REFRESH, SPARSE, DetailBank, Operator, SparseAttention
from .host_banks import HostBankOperator

__all__ = [
    "EXACT", "REFRESH", "SPARSE", "DetailBank", "HostBankOperator", "Layout", "OperatingPoint",
    "Operator", "OperatorConfig", "RecapConfig", "SparseAttention", "SparseGeometry",
    "config_from_dict", "hilbert_permutation", "load_config",
]
