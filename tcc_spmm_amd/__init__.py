"""tcc_spmm_amd — MI355X-native TCC-SpMM: Y = A x tf32(dequant(X_int8)) on gfx950.

Host format (CPU): make_canonical_csr, load_matrix_market, convert_csr_to_sw32, Sw32HostFormat.
Device (HIP via libtcc_spmm.so, module tcc_spmm_amd.device): quantize_features_int8,
pack_features_int8x16, launch_spmm_int8, TorchDeviceMatrix / NativeDeviceMatrix; and, with no
counterpart in the original library, quantize_pack_features_int8 (both feature steps in one pass)
and launch_spmm_int8_noalloc (no caller workspace). torch is imported lazily, only by the device
module.
"""
from .format import (NO_PARTIAL, SW32_BUCKET_ORDER, SW32_TASK_PANEL_LIMIT, CsrMatrix,
                     Sw32HostFormat, convert_csr_to_sw32, csr_from_arrays, load_matrix_market, make_canonical_csr,
                     synth_csr, synth_features)

__all__ = [
    "NO_PARTIAL", "SW32_BUCKET_ORDER", "SW32_TASK_PANEL_LIMIT", "CsrMatrix", "Sw32HostFormat",
    "convert_csr_to_sw32", "csr_from_arrays", "load_matrix_market", "make_canonical_csr", "synth_csr",
    "synth_features",
]
