"""janas_amd - KV-cache attention for MI355X (gfx950) behind the engine's C
attention interface. The product is libjanas_attn.so (include/janas_attn.h);
this package builds it (``janas_amd.build``) and mirrors its interface in
Python (``janas_amd.attention``)."""
from .attention import (AUTO, EDEVICE, EINVAL, ENOMEM, ENOTSUP, ERANGE, FLOAT,
                        GATE_ELEM, GATE_HEAD, GATE_NONE, INT16, KV_F16,
                        KV_F32, KV_I8, KV_I16, MAX_BLOCK, OK, Attention,
                        AttnError, lib, part_bytes, ring_positions, strerror)

__all__ = ["AUTO", "FLOAT", "INT16", "KV_I8", "KV_I16", "KV_F16", "KV_F32",
           "OK", "EINVAL", "ERANGE", "ENOMEM", "EDEVICE", "ENOTSUP",
           "GATE_NONE", "GATE_ELEM", "GATE_HEAD", "MAX_BLOCK", "Attention",
           "AttnError", "lib", "part_bytes", "ring_positions", "strerror"]
