from .attention import HIPBailingMoEAttention
from .decoder_layer import HIPBailingMoEDecoderLayer
from .kv_cache import HIPPagedAttentionKVCache, PagedAttentionConfig
from .model import HIPBailingMoeV2Model, HIPLMHead
from .moe import HIPBailingMoE, HIPBailingMoeV2MLP

__all__ = ["HIPBailingMoEAttention", "HIPBailingMoEDecoderLayer", "HIPPagedAttentionKVCache",
           "PagedAttentionConfig", "HIPBailingMoE", "HIPBailingMoeV2MLP",
           "HIPBailingMoeV2Model", "HIPLMHead"]
