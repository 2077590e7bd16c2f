"""gfx950 (MI355X) attention path for nano-inference.

Hand-written HIP kernels behind a C ABI (libnia_attn.so, include/nia_attn.h),
with PyTorch-side layers that keep the reference engine's attention interface:

* ``ops``        - tensor-level wrappers of the C ABI (kv_write, paged_decode,
                   prefill, varlen_attention, prefill_paged, and the fused
                   qk_norm_rope_kv_write that feeds them);
* ``attention``  - ``PagedCausalSelfAttention``, ``Qwen25VLDecoderAttention`` and
                   ``scaled_dot_product_attention`` as drop-ins for
                   src/nano_inference/layers/attention.py;
* ``vision``     - ``VisionAttention`` (Qwen2.5-VL ViT) and its chunk producers;
* ``context``    - ``AttentionMetadata`` and ``GenerateContext``, field-for-field the
                   reference's;
* ``context_builder`` - ``GenerateContextBuilder``: the step's inputs and metadata
                   built on the GPU from one upload (``nia_step_metadata``);
* ``e2e``        - a Qwen3-architecture decoder over these layers with a paged KV
                   pool and a batched greedy generator (whole-model throughput).
"""
from . import _lib, ops  # noqa: F401
from .attention import (  # noqa: F401
    PagedCausalSelfAttention,
    Qwen25VLDecoderAttention,
    scaled_dot_product_attention,
)
from .context import AttentionMetadata, GenerateContext  # noqa: F401
from .context_builder import GenerateContextBuilder, select_last_logits  # noqa: F401
from .vision import VisionAttention, full_cu_seqlens, window_index  # noqa: F401

__all__ = [
    "ops",
    "AttentionMetadata",
    "GenerateContext",
    "GenerateContextBuilder",
    "select_last_logits",
    "PagedCausalSelfAttention",
    "Qwen25VLDecoderAttention",
    "scaled_dot_product_attention",
    "VisionAttention",
    "full_cu_seqlens",
    "window_index",
]
