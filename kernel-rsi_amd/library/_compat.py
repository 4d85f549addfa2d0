"""Eager / torch.compile dispatch for the library kernels.

Two paths over the same HIP kernels, chosen per call by the public function
(the same split the reference makes in library/_compat.py:1-27):
- under torch.compile: a `torch.library.custom_op` ("krsi::...") with a fake
  (meta) implementation and `register_autograd`, so dynamo traces it as one
  opaque operator (fullgraph=True works, no graph break);
- in eager: a plain `torch.autograd.Function` that calls the ctypes launchers
  directly, which skips the dispatcher's per-call host cost.
"""
import torch

HAS_CUSTOM_OP = hasattr(torch.library, "custom_op") and hasattr(torch.library, "register_fake")


def compiling() -> bool:
    """True while dynamo is tracing (use the registered op), else eager."""
    return HAS_CUSTOM_OP and torch.compiler.is_compiling()
