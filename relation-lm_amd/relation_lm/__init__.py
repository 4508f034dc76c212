"""Relation LM routed relation path, MI355X (gfx950) native.

Drop-in for the reference package's hot path: ``relation_lm.kernels`` and
``relation_lm.inference`` keep the reference's module paths, function names
and ``torch.ops`` schemas, backed by hand-written HIP kernels in
``_lib/librlm_hip.so`` (C ABI, ``include/relation_lm_hip.h``) and registered by
``_lib/_rlm_torch.so``.
"""

__version__ = "0.1.0"
