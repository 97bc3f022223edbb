"""The reference's import name for this build: `import aneforge as af` and `from aneforge.llm import
...` resolve to aneforge_amd and its modules, so code written against the reference
(aneforge/__init__.py:13-38) runs unchanged on the MI355X path."""
import importlib as _importlib
import sys as _sys

import aneforge_amd as _impl
from aneforge_amd import *  # noqa: F401,F403
from aneforge_amd import __all__, __version__  # noqa: F401

# the reference's module names on this path, each the same module object as aneforge_amd's
for _name in ("graph", "llm", "moe", "speculative", "_gguf", "_blob", "_compile", "_runtime"):
    _mod = _importlib.import_module(f"aneforge_amd.{_name}")
    _sys.modules[f"{__name__}.{_name}"] = _mod
    globals()[_name] = _mod
del _name, _mod
