"""Import shim: loads the package directory ``minicpm-o-4.5-single-gpu-engine_amd/`` (not a valid Python identifier)
as the importable package ``t2w_amd``."""

import importlib.util
import pathlib
import sys

_DIR = pathlib.Path(__file__).resolve().with_name("minicpm-o-4.5-single-gpu-engine_amd")
_spec = importlib.util.spec_from_file_location(__name__, _DIR / "__init__.py", submodule_search_locations=[str(_DIR)])
_mod = importlib.util.module_from_spec(_spec)
sys.modules[__name__] = _mod
_spec.loader.exec_module(_mod)
