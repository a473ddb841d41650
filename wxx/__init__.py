"""The reference's import name for this backend: ``import wxx`` gives the
``wxx_amd`` package, and every ``wxx.<sub>`` module path (for example
``from wxx.functional.utils import from_numpy``, reference
src/wxx/nn/module.py:5) resolves to the same module object as
``wxx_amd.<sub>``, so code written against the reference runs unchanged and
both names share one device, one allocator and one set of classes.
"""

import importlib
import importlib.abc
import importlib.util
import sys

import wxx_amd as _impl

_ALIAS, _TARGET = "wxx", "wxx_amd"


class _AliasLoader(importlib.abc.Loader):
    def __init__(self, target):
        self._target = target

    def create_module(self, spec):
        return importlib.import_module(self._target)

    def exec_module(self, module):
        # the target module is already initialised by its own import
        pass


class _AliasFinder(importlib.abc.MetaPathFinder):
    def find_spec(self, fullname, path=None, target=None):
        if not fullname.startswith(_ALIAS + "."):
            return None
        real = _TARGET + fullname[len(_ALIAS):]
        if importlib.util.find_spec(real) is None:
            return None
        mod = importlib.import_module(real)
        spec = importlib.util.spec_from_loader(fullname, _AliasLoader(real),
                                               is_package=hasattr(mod, "__path__"))
        return spec


if not any(isinstance(f, _AliasFinder) for f in sys.meta_path):
    sys.meta_path.insert(0, _AliasFinder())

# ``import wxx`` binds the implementation package itself (same attributes,
# same submodule objects).
sys.modules[__name__] = _impl
