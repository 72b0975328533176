"""MI355X-native blockwise-sparse NF4 MLP decode (gfx950 HIP kernels + C ABI).

Modules:
  sparse_mlp  drop-in replacements for the reference's sparse-MLP kernel
              entry points (same names and signatures)
  router      the learned-basis router on the GPU (route_sparse_mlp)
  slot_table  the HBM hot-block slot table and the one-call decode layer
  layout      block-bank layout contract and the active-block layout
  synth       seeded synthetic NF4 layers generated on the GPU
"""
from .layout import (  # noqa: F401
    MlpBlockBankLayout,
    build_intermediate_mlp_block_bank_layout,
    build_sparse_active_layout,
    validate_intermediate_mlp_block_bank_params,
)

__version__ = "0.1.0"
