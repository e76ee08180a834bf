"""mkx: MI355X-native persistent megakernel for the Euler loop of a flow-matching DiT action expert.

``ExpertMegakernel`` / ``install`` mirror the reference's expert-call boundary (src/mk_expert.py:433-536);
``synthetic`` holds the REKI-shaped random-init expert the kernel is measured on.
"""
from .mk_expert import ExpertMegakernel, install  # noqa: F401
from . import synthetic  # noqa: F401

__all__ = ["ExpertMegakernel", "install", "synthetic"]
