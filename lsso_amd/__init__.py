"""MI355X-native LSSO: the DYNAMIC + Rank-Rotary token mixer on gfx950.

Public surface mirrors the reference package ``lsso`` (lsso/__init__.py:1-7):
``CoreMode``, ``LSSO``, ``LSSOConfig`` and ``__version__``.
"""

from .ball import CoreMode, LSSO, LSSOConfig

__version__ = "0.6.3"

__all__ = ["CoreMode", "LSSO", "LSSOConfig", "__version__"]
