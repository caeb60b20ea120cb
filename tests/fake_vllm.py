"""A minimal stand-in for the parts of vLLM the AMASS backend touches (vLLM is not
installable here).  ``install()`` puts modules into sys.modules that mimic the ROCm
platform's backend selection, one decoder attention backend (impl + metadata builder),
AttentionCGSupport and the config objects the builder reads."""
from __future__ import annotations

import dataclasses
import enum
import sys
import types

TRITON_PATH = "vllm.v1.attention.backends.triton_attn.TritonAttentionBackend"
MLA_PATH = "vllm.v1.attention.backends.mla.rocm_aiter_mla.AiterMLABackend"


class AttentionCGSupport(enum.Enum):
    ALWAYS = 3
    UNIFORM_BATCH = 2
    UNIFORM_SINGLE_TOKEN_DECODE = 1
    NEVER = 0


class AttentionType:
    DECODER = "decoder"
    ENCODER = "encoder"


class TritonAttentionImpl:
    def __init__(self, num_heads, head_size, scale, num_kv_heads):
        self.num_heads, self.head_size, self.scale = num_heads, head_size, scale
        self.num_kv_heads = num_kv_heads
        self.attn_type = AttentionType.DECODER
        self.sliding_window = (-1, -1)
        self.alibi_slopes = None
        self.sinks = None
        self.kv_cache_dtype = "auto"
        self.calls = []

    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None,
                output_scale=None, output_block_scale=None):
        self.calls.append("stock")
        return output


class Metadata(types.SimpleNamespace):
    pass


class TritonAttentionMetadataBuilder:
    def __init__(self, kv_cache_spec, layer_names, vllm_config, device):
        self.kv_cache_spec, self.layer_names = kv_cache_spec, layer_names
        self.vllm_config, self.device = vllm_config, device

    def build(self, common_prefix_len, common_attn_metadata, fast_build=False):
        cam = common_attn_metadata
        return Metadata(seq_lens=cam.seq_lens, block_table=cam.block_table_tensor,
                        max_query_len=cam.max_query_len, causal=True,
                        query_start_loc=getattr(cam, "query_start_loc", None),
                        slot_mapping=getattr(cam, "slot_mapping", None),
                        num_actual_tokens=getattr(cam, "num_actual_tokens", None))

    def build_for_cudagraph_capture(self, common_attn_metadata):
        return self.build(0, common_attn_metadata)


class TritonAttentionBackend:
    @staticmethod
    def get_name():
        return "TRITON_ATTN"

    @staticmethod
    def get_impl_cls():
        return TritonAttentionImpl

    @staticmethod
    def get_builder_cls():
        return TritonAttentionMetadataBuilder


class RocmPlatform:
    @classmethod
    def get_attn_backend_cls(cls, selected_backend, head_size, dtype, kv_cache_dtype,
                             block_size, use_v1=True, use_mla=False, **kw):
        return MLA_PATH if use_mla else TRITON_PATH


@dataclasses.dataclass(frozen=True)
class FullAttentionSpec:
    block_size: int
    num_kv_heads: int
    head_size: int
    head_size_v: int


@dataclasses.dataclass(frozen=True)
class SlidingWindowSpec:
    block_size: int
    num_kv_heads: int
    head_size: int
    sliding_window: int


class Attention:
    """The attention layer: get_kv_cache_spec as vLLM's layer returns it."""

    def __init__(self, spec):
        self.spec = spec

    def get_kv_cache_spec(self, vllm_config):
        return self.spec


def vllm_config(*, num_gpu_blocks, layers, max_num_seqs=4, max_model_len=4096,
                n_q=32):
    sfc = {name: types.SimpleNamespace(kv_cache=[kv]) for name, kv in layers.items()}
    return types.SimpleNamespace(
        cache_config=types.SimpleNamespace(num_gpu_blocks=num_gpu_blocks),
        compilation_config=types.SimpleNamespace(static_forward_context=sfc),
        scheduler_config=types.SimpleNamespace(max_num_seqs=max_num_seqs),
        model_config=types.SimpleNamespace(max_model_len=max_model_len,
                                           num_attention_heads=n_q),
        parallel_config=None)


def kv_spec(n_kv=8, head_size=128, block_size=16):
    return types.SimpleNamespace(num_kv_heads=n_kv, head_size=head_size,
                                 block_size=block_size)


def install():
    mods = {}

    def mod(name, **attrs):
        m = types.ModuleType(name)
        m.__dict__.update(attrs)
        mods[name] = m
        return m

    mod("vllm")
    mod("vllm.platforms", rocm=None)
    rocm = mod("vllm.platforms.rocm", RocmPlatform=RocmPlatform)
    mods["vllm.platforms"].rocm = rocm
    mod("vllm.v1")
    mod("vllm.v1.attention")
    mod("vllm.v1.attention.backend", AttentionCGSupport=AttentionCGSupport,
        AttentionType=AttentionType)
    mod("vllm.v1.attention.backends")
    mod("vllm.attention")
    mod("vllm.attention.layer", Attention=Attention)
    mod("vllm.v1.attention.backends.triton_attn", TritonAttentionBackend=TritonAttentionBackend,
        TritonAttentionImpl=TritonAttentionImpl,
        TritonAttentionMetadataBuilder=TritonAttentionMetadataBuilder)
    saved = {k: sys.modules.get(k) for k in mods}
    sys.modules.update(mods)
    return saved


def uninstall(saved):
    for k, v in saved.items():
        if v is None:
            sys.modules.pop(k, None)
        else:
            sys.modules[k] = v
