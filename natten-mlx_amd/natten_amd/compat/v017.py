"""NATTEN v0.17 API: identical to v0.15 (``compat/v017.py:1-3``)."""

from .v015 import *  # noqa: F401,F403
from .v015 import __all__  # noqa: F401
