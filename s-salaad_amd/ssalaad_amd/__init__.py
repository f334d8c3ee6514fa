"""MI355X (gfx950) sparse-plus-low-rank linear: y = x·Bᵀ·Aᵀ + x·Sᵀ + b.

Drop-in for the S-SALAAD hot path:
  * torch.ops.ssalaad.tilelang_bsr_addmm_inplace_dense_  (ssalaad_amd.addmm_inplace)
  * LRSLinear                                              (ssalaad_amd.ls_linear)
  * LRSLinearGroup: linears sharing an input in one launch (ssalaad_amd.ls_linear)
  * LRSLinearChain: dependent stages of linears in one launch (ssalaad_amd.ls_linear)
  * dense_to_bsr / factor_from_svd                         (ssalaad_amd.artifact)
  * project_S / project_S_nm: the compression loop's sparse steps (ssalaad_amd.project)
  * save_artifact / load_artifact / build_efficient_model: bundles (ssalaad_amd.bundle)
  * DecodeEngine / generate: KV-cached greedy decode of a loaded model (ssalaad_amd.decode)
All compute runs in the HIP kernels of libssalaad_amd.so; there is no CPU path.
"""

from __future__ import annotations

from . import _lib
from .addmm_inplace import (SUPPORTED_BLOCK_SIZES, bsr_addmm_inplace_, get_tuned_config,
                            prepare_bsr_addmm)
from .artifact import dense_to_bsr, encode_for_kernels, factor_from_svd
from .bundle import build_efficient_model, load_artifact, save_artifact
from .decode import DecodeEngine, generate
from .ls_linear import (LRSLinear, LRSLinearChain, LRSLinearGroup, PreparedChain,
                        clear_wait_status, latent_wait_status)
from .project import block_topk, project_S, project_S_nm, project_nm

__all__ = [
    "DecodeEngine",
    "LRSLinear",
    "LRSLinearChain",
    "LRSLinearGroup",
    "PreparedChain",
    "SUPPORTED_BLOCK_SIZES",
    "block_topk",
    "build_efficient_model",
    "bsr_addmm_inplace_",
    "clear_wait_status",
    "prepare_bsr_addmm",
    "dense_to_bsr",
    "encode_for_kernels",
    "factor_from_svd",
    "generate",
    "get_tuned_config",
    "latent_wait_status",
    "library_path",
    "load_artifact",
    "project_S",
    "project_S_nm",
    "project_nm",
    "save_artifact",
]


def library_path() -> str:
    return str(_lib.LIB_PATH)
