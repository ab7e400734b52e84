"""Import name of the package in ``qwen3.8-flash-next-24gb-sglang_amd/`` (a directory name that is not a Python
identifier): ``import kvtier`` loads that directory as the package ``kvtier``."""
import importlib.util
import os
import sys

_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "qwen3.8-flash-next-24gb-sglang_amd")
_spec = importlib.util.spec_from_file_location(__name__, os.path.join(_DIR, "__init__.py"),
                                               submodule_search_locations=[_DIR])
_mod = importlib.util.module_from_spec(_spec)
sys.modules[__name__] = _mod
_spec.loader.exec_module(_mod)
