"""sglang_neuron_amd: sglang-neuron's paged decode-attention path, rebuilt for MI355X (gfx950).

The package mirrors the reference plugin's attention-backend and KV-pool API (``attention.backend``,
``mem_cache.memory_pool``) and runs every kernel through the C ABI of libsglang_neuron_amd.so (``ops``). The Python
package name is the importable spelling of ``sglang-neuron_amd``.
"""

__version__ = "0.1.0"
