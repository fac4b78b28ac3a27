"""Layer API mirroring the reference's ``looped_blockell.layers`` (Block-ELL format, MLP, RMSNorm)."""

from .block_ell import (BlockELLConfig, BlockELLTensor, block_ell_matmul, block_ell_to_dense,
                        create_block_ell_from_dense, create_random_topology)
from .looped import LoopedCore, LoopedSwiGLU
from .mlp import BlockELLLinear, MLPBlock
from .norms import RMSNorm
from .ternary import TernaryBlockELLWeight, TernaryMLPBlock

__all__ = [
    "BlockELLConfig", "BlockELLTensor", "block_ell_matmul", "block_ell_to_dense", "create_block_ell_from_dense",
    "create_random_topology", "BlockELLLinear", "MLPBlock", "RMSNorm", "LoopedSwiGLU", "LoopedCore", "TernaryBlockELLWeight",
    "TernaryMLPBlock",
]
