"""Drop-in alias: ``import spira`` resolves to :mod:`spira_amd`, so scripts
written against the reference package (source/spira/__init__.py:1-6) run
unchanged -- ``spira.SparseTensor``, ``spira.nn.SparseConv``,
``spira.nn.functional.build_kmap``, ``spira.tune`` and the rest refer to the
MI355X implementation.  Every submodule of spira_amd is registered under the
same dotted name below ``spira``."""
import importlib
import pkgutil
import sys

import spira_amd as _impl

_pkg = sys.modules[__name__]
for _info in pkgutil.walk_packages(_impl.__path__, prefix="spira_amd."):
    if _info.name.startswith("spira_amd.csrc") or _info.name == "spira_amd.build":
        continue
    try:
        _mod = importlib.import_module(_info.name)
    except ImportError:
        # the native extension is missing: spira_amd.nn.functional raises on
        # import and so does spira.nn.functional, with the same message
        continue
    sys.modules["spira" + _info.name[len("spira_amd"):]] = _mod

sys.modules[__name__] = _impl
