"""HIP (gfx950) kernels of the routed relation path.

Module names follow the reference package (``relation_select``,
``triton_select``, ``relation_reduce``) so existing imports keep working; the
kernels themselves are hand-written HIP, not Triton.
"""
