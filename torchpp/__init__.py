"""Drop-in alias: `import torchpp.X` resolves to `torchplusplus_amd.X`, so code
written against the reference package (e.g. examples/LLM/fastqwen3.py:7-11,
`from torchpp.dlops.normalization import RmsNormFused`) runs unchanged on the
gfx950 implementation."""
import importlib
import importlib.abc
import importlib.util
import sys

import torchplusplus_amd as _impl

_PREFIX = __name__ + "."


class _AliasLoader(importlib.abc.Loader):
    def __init__(self, target):
        self.target = target

    def create_module(self, spec):
        return importlib.import_module(self.target)

    def exec_module(self, module):
        pass


class _AliasFinder(importlib.abc.MetaPathFinder):
    def find_spec(self, name, path=None, target=None):
        if not name.startswith(_PREFIX):
            return None
        real = "torchplusplus_amd." + name[len(_PREFIX):]
        if importlib.util.find_spec(real) is None:
            return None
        return importlib.util.spec_from_loader(name, _AliasLoader(real))


if not any(isinstance(f, _AliasFinder) for f in sys.meta_path):
    sys.meta_path.insert(0, _AliasFinder())

__version__ = _impl.__version__
