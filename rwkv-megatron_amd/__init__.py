"""MI355X-native RWKV-6 time-mix hot path (drop-in for RWKV-Megatron's fla call).

The package directory name carries a dash, so load it with
``importlib.import_module("rwkv-megatron_amd")``.

Exports
  chunk_rwkv6, fused_recurrent_rwkv6   fla-compatible WKV6 ops (wkv.py, HIP kernels)
  wkv6_seqfirst                        WKV6 on the time-mix module's [T,B,H*64] layout
  timemix                              fused token-shift/ddlerp and GroupNorm*gate ops
  channelmix                           fused channel-mix shift/lerp, relu^2, sigmoid gate
  modules                              RWKV6TimeMix / RWKV6ChannelMix / ... mirrors of
                                       rwkv_megatron/rwkv6_layer_specs.py
"""
from .wkv import chunk_rwkv6, fused_recurrent_rwkv6, wkv6_seqfirst  # noqa: F401
from . import _lib, channelmix, timemix, modules  # noqa: F401

__all__ = ["chunk_rwkv6", "fused_recurrent_rwkv6", "wkv6_seqfirst", "timemix", "channelmix", "modules"]
