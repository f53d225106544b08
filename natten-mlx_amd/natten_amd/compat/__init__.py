"""Historical NATTEN API surfaces (mirrors ``compat/__init__.py:1-25``).

``for_version("0.14.6")`` returns the module that reproduces that NATTEN
release's Python API on top of this package: v0.14 and older -> ``v014``,
up to 0.15 -> ``v015``, up to 0.17 -> ``v017``, anything newer -> ``v020``.
"""

from __future__ import annotations

from importlib import import_module

from packaging.version import Version


def for_version(version: str):
    """Compat module for a NATTEN version string (``compat/__init__.py:9-22``);
    an unparsable string raises ``packaging.version.InvalidVersion``."""
    v = Version(version)
    target = (v.major, v.minor)
    if target <= (0, 14):
        name = "v014"
    elif target <= (0, 15):
        name = "v015"
    elif target <= (0, 17):
        name = "v017"
    else:
        name = "v020"
    return import_module(f"{__name__}.{name}")


__all__ = ["for_version"]
