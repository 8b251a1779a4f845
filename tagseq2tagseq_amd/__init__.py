"""gfx950 (MI355X) masked flash-attention path of tagseq2tagseq.

Public surface (mirrors the reference's seams):
  mask creators   -- tagseq2tagseq_amd.mask_creators
  BlockMask       -- tagseq2tagseq_amd.block_mask.T2TBlockMask
  attention       -- tagseq2tagseq_amd.attention.flex_attention / FlexSelfAttention
"""
from .block_mask import T2TBlockMask, build_block_mask  # noqa: F401
from .attention import FlexSelfAttention, T2TFlexAttentionFn, flex_attention  # noqa: F401
from .mask_creators import (  # noqa: F401
    MASK_CREATORS,
    CrossDocLinkMaskCreator,
    create_causal_block_mask,
    create_doc_causal_block_mask,
    create_doc_link_block_mask,
    get_mask_creator,
    list_mask_creators,
    make_mask_creator_callable,
    make_mask_creator_callable_from,
)

__version__ = "0.1.0"
