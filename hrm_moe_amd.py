"""Import shim: ``import hrm_moe_amd`` loads the package kept in ``hrm-moe_amd/``.

The package directory name contains a hyphen, which Python's import
statement cannot name.  This module loads that directory as the package
``hrm_moe_amd`` and puts it in ``sys.modules`` in place of itself.
"""
import importlib.util
import os
import sys

_PKG_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "hrm-moe_amd")
_spec = importlib.util.spec_from_file_location("hrm_moe_amd", os.path.join(_PKG_DIR, "__init__.py"),
                                               submodule_search_locations=[_PKG_DIR])
_module = importlib.util.module_from_spec(_spec)
sys.modules["hrm_moe_amd"] = _module
_spec.loader.exec_module(_module)
