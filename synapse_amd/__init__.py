"""synapse_amd — MI355X (gfx950) KV-cache attention for synapse.

The product is the C ABI in include/synapse_hip.h, implemented by the HIP
kernels under csrc/ and built into libsynapse_hip.so; host/ holds the C++20
graph builder, planner and session that call it. This Python package only
builds the library and binds it with ctypes (for tests and the benchmark).
"""
from .capi import (SYN_F16, SYN_F32, Arena, AttnDesc, KvDesc, RopeDesc, SelfDesc, SeqDesc, SynHipError, check,
                   kv_state, lib)

__all__ = ["SYN_F16", "SYN_F32", "Arena", "AttnDesc", "KvDesc", "RopeDesc", "SelfDesc", "SeqDesc", "SynHipError",
           "check", "kv_state", "lib"]
