"""`import enceladus` for drop-in user code: an alias of the MI355X backend package.

Existing kernels keep `import enceladus`, `import enceladus.language as tl` and imports of
submodules such as `from enceladus.compiler.errors import CompilationError`. Every
`enceladus.X` resolves to the module object `enceladus_amd.X` itself (a finder on
`sys.meta_path` hands out the existing module rather than loading a second copy), so
classes, `isinstance` checks and `except` clauses agree whichever name imported them.
"""

import importlib
import importlib.abc
import importlib.util
import sys

_ALIAS = __name__
_TARGET = "enceladus_amd"


class _AliasLoader(importlib.abc.Loader):
    def __init__(self, module):
        self.module = module

    def create_module(self, spec):
        return self.module

    def exec_module(self, module):
        pass                                    # already executed under its own name


class _AliasFinder(importlib.abc.MetaPathFinder):
    """Finds `enceladus.X` by importing `enceladus_amd.X` and returning that module."""

    def find_spec(self, fullname, path=None, target=None):
        if not fullname.startswith(_ALIAS + "."):
            return None
        real = _TARGET + fullname[len(_ALIAS):]
        try:
            module = importlib.import_module(real)
        except ModuleNotFoundError as e:
            if e.name == real:
                return None                     # no such submodule: a normal ImportError
            raise
        return importlib.util.spec_from_loader(fullname, _AliasLoader(module),
                                               is_package=hasattr(module, "__path__"))


if not any(isinstance(f, _AliasFinder) for f in sys.meta_path):
    sys.meta_path.insert(0, _AliasFinder())

import enceladus_amd as _pkg  # noqa: E402

sys.modules[_ALIAS] = _pkg
# submodules already imported under their real names are registered under the alias too
for _name, _mod in list(sys.modules.items()):
    if _name.startswith(_TARGET + ".") and _mod is not None:
        sys.modules.setdefault(_ALIAS + _name[len(_TARGET):], _mod)
