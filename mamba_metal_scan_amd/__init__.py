"""MI355X-native fused selective scan for Mamba (gfx950 HIP kernels).

Same public surface as the reference package ``mamba_metal``
(mamba_metal/__init__.py:2-7), plus the HIP-specific names.
"""
from .conv import ConvSiluHIP, conv1d_silu
from .fused import (MambaInnerHIP, OutGateHIP, SelectiveScanGatedHIP, mamba_inner, out_gate,
                    selective_scan_gated)
from .model import MambaConfig, TinyMamba
from .norm import AddRMSNormHIP, RMSNormHIP, add_rms_norm, rms_norm, rms_norm_residual
from .xent import CrossEntropyHIP, cross_entropy
from .scan import (SSM_CHUNK, SelectiveScanHIP, selective_scan, selective_scan_hip,
                   selective_scan_metal, selective_scan_ref, selective_state_step)

__all__ = ["MambaConfig", "TinyMamba", "SSM_CHUNK", "SelectiveScanHIP", "selective_scan",
           "selective_scan_hip", "selective_scan_metal", "selective_scan_ref",
           "selective_state_step", "conv1d_silu", "ConvSiluHIP", "selective_scan_gated",
           "SelectiveScanGatedHIP", "out_gate", "OutGateHIP", "mamba_inner", "MambaInnerHIP",
           "cross_entropy", "CrossEntropyHIP", "rms_norm", "rms_norm_residual", "RMSNormHIP",
           "add_rms_norm", "AddRMSNormHIP"]
