"""needle_amd: MI355X-native paged-KV hot path for the Needle inference engine.

The operations live in needle_amd.ops (torch tensors in, HIP kernels through
the C ABI of include/needle_amd.h); needle_amd.layers.attention.Attention is
the drop-in for needle/layers/attention.py:Attention.
"""
__version__ = "0.1.0"
