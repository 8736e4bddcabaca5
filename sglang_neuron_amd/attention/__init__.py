"""The attention backend of the HIP decode path (the reference's sglang_neuron/attention/backend.py interface)."""

from .backend import NeuronAttnBackend, NeuronForwardMetadata

__all__ = ["NeuronAttnBackend", "NeuronForwardMetadata"]
