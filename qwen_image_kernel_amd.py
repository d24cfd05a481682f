"""Import shim: ``import qwen_image_kernel_amd`` loads the package directory
``qwen-image-kernel_amd/`` (a directory name Python cannot import directly) and
registers it under this module name, so its submodules import normally
(``qwen_image_kernel_amd.attention``, ``qwen_image_kernel_amd.kv_cache``, ...)."""

import importlib.util
import os
import sys

_PKG_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "qwen-image-kernel_amd")
_spec = importlib.util.spec_from_file_location(
    __name__, os.path.join(_PKG_DIR, "__init__.py"), submodule_search_locations=[_PKG_DIR]
)
_mod = importlib.util.module_from_spec(_spec)
sys.modules[__name__] = _mod
_spec.loader.exec_module(_mod)
