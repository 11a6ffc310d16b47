"""ternel_amd -- MI355X (gfx950) execution engine for TQ1_G128 packed ternary weights.

Public surface mirrors the reference's packed-linear path:
``PackedTensorLayout`` (layout), ``PackedLinear`` / ``PackedEmbedding`` /
``packed_matmul`` (modules), ``tq1_matmul`` / ``tq1_gemm`` / ``tq1_get_rows``
(kernels), ``encode_tq1_blocks`` / ``decode_tq1_blocks`` / ``FormatError``
(format). All compute runs in ``_lib/libternel_tq1.so`` (hand-written HIP for
gfx950, C ABI in include/ternel_tq1.h).
"""

from .format import (
    BLOCK_BYTES,
    BLOCK_SIZE,
    MAX_FULL_CODE_BYTE,
    MAX_TAIL_CODE_BYTE,
    FormatError,
    decode_tq1_blocks,
    encode_tq1_blocks,
    validate_blocks,
    validate_packed_codes,
)
from .kernels import (GemmConfig, MatmulConfig, tq1_gemm, tq1_gemm_words, tq1_get_rows, tq1_get_rows_words,
                      tq1_linear_words, tq1_matmul, tq1_matmul_words)
from .layout import PackedTensorLayout, pack_blocks, select_tile, unpack_blocks
from .modules import PackedEmbedding, PackedLinear, packed_matmul, replace_with_packed

__version__ = "0.3.0"
