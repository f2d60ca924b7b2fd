"""helios_amd: an MI355X-native (gfx950) paged-attention path for helios.

The public surface mirrors ``helios.exec.paged_attn`` (PagedKVCache,
QuantizedPagedKVCache, paged_attention_decode, paged_attention_decode_batched,
paged_attention_prefill) and adds the batched and raw-tensor forms.  The
compute lives in ``libheliosattn.so`` (C-ABI: include/helios_attn.h), built
by ``python -m helios_amd.build``.
"""

from .paged_attn import (  # noqa: F401
    PagedKVCache,
    QuantizedPagedKVCache,
    _repeat_kv,
    _repeat_kv_batched,
    copy_blocks,
    decode_workspace,
    decode_workspace_bytes,
    hip_available,
    paged_attention_decode,
    paged_attention_decode_batched,
    paged_attention_decode_hip,
    paged_attention_prefill,
    paged_attention_varlen,
    paged_attention_verify_batched,
    reset_decode_workspace,
    write_kv,
)
from .step_meta import DeviceAttnMeta, DeviceBlockTables, batched_attention, write_kv_batched  # noqa: F401

__all__ = [
    "PagedKVCache",
    "QuantizedPagedKVCache",
    "copy_blocks",
    "decode_workspace",
    "decode_workspace_bytes",
    "hip_available",
    "paged_attention_decode",
    "paged_attention_decode_batched",
    "paged_attention_decode_hip",
    "paged_attention_prefill",
    "paged_attention_varlen",
    "paged_attention_verify_batched",
    "reset_decode_workspace",
    "write_kv",
    "DeviceAttnMeta",
    "DeviceBlockTables",
    "batched_attention",
    "write_kv_batched",
]
