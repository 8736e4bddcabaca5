"""KV pools of the HIP decode path (the reference's sglang_neuron/mem_cache/memory_pool.py interface)."""

from .memory_pool import (NeuronDSATokenToKVPool, NeuronMHATokenToKVPool, NeuronMHATokenToKVPoolKind,
                          NeuronMLATokenToKVPool, full_attention_pool)

__all__ = ["NeuronMHATokenToKVPool", "NeuronMHATokenToKVPoolKind", "NeuronMLATokenToKVPool", "NeuronDSATokenToKVPool",
           "full_attention_pool"]
