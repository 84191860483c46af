"""Drop-in import name of the reference package (``import fastgs_core``).

Re-exports the MI355X implementation in ``fastgs_core_amd``, as the
reference package re-exports its extension module
(python_package/fastgs_core/__init__.py:1-2).
"""
from fastgs_core_amd import *  # noqa: F401,F403
from fastgs_core_amd import __all__  # noqa: F401
