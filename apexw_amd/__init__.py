"""apexw_amd: MI355X-native (gfx950) fused optimizer step for ApexW.

Drop-in host API (``ApexW``, ``HybridApexW``, ``ApexMuon``) over hand-written
HIP kernels in ``libapexw_hip.so`` (built in-tree by ``apexw_amd._build``).
"""

from .optimizer import ApexW
from .muon import ApexMuon
from .hybrid import HybridApexW, partition_parameters_for_hybrid

__version__ = "0.1.0"
__all__ = ["ApexW", "ApexMuon", "HybridApexW", "partition_parameters_for_hybrid"]
