"""The reference's import name, ``cublade``, for the MI355X build.

User code written against emre570/cublade imports ``cublade.quantization``,
``cublade.bindings.cuda.<module>`` and ``cublade._loader`` (reference:
cublade/__init__.py:1-6, cublade/bindings/__init__.py:1-2,
cublade/bindings/cuda/__init__.py:1-4, cublade/_loader.py:24-125). Every such
module here IS the corresponding module of ``cublade_amd`` (the same module
object, so state such as the loader's memo is shared):

    cublade.<sub>                 ->  cublade_amd.<sub>
    cublade.bindings.cuda[.<m>]   ->  cublade_amd.bindings.hip[.<m>]

The mapping is done by an import hook, so submodules that are imported lazily
(``cublade.benchmark.suite``, ``cublade.quantization.linear`` ...) resolve the
same way. Names with no counterpart on the quantization path (the Triton
bindings, ``cublade.kernels``, ``avg_pool_1d``) raise ImportError.

The top-level namespace re-exports what the reference's star imports put
there for this path: the quantization API and the HIP binding functions.
The first-import warm-up (``CUBLADE_SKIP_WARMUP``) is the one of
``cublade_amd``.
"""
from __future__ import annotations

import importlib
import importlib.abc
import importlib.util
import sys

_IMPL = "cublade_amd"
# Reference subpackage name -> implementation subpackage name.
_RENAMES = (("bindings.cuda", "bindings.hip"),)


def _target(fullname: str) -> str | None:
    """Implementation module for a ``cublade.<rest>`` name, or None."""
    if not fullname.startswith(__name__ + "."):
        return None
    rest = fullname[len(__name__) + 1:]
    for ref, impl in _RENAMES:
        if rest == ref or rest.startswith(ref + "."):
            rest = impl + rest[len(ref):]
            break
    return f"{_IMPL}.{rest}"


class _AliasLoader(importlib.abc.Loader):
    """Hands out the already-imported implementation module under the alias
    name, without executing anything a second time."""

    def __init__(self, target: str):
        self._target = target
        self._spec = None

    def create_module(self, spec):
        module = importlib.import_module(self._target)
        self._spec = module.__spec__
        return module

    def exec_module(self, module):
        # importlib sets module.__spec__ to the alias spec; keep the real one.
        module.__spec__ = self._spec


class _AliasFinder(importlib.abc.MetaPathFinder):
    def find_spec(self, fullname, path=None, target=None):
        impl = _target(fullname)
        if impl is None:
            return None
        if importlib.util.find_spec(impl) is None:
            return None
        return importlib.util.spec_from_loader(fullname, _AliasLoader(impl),
                                               is_package=_is_package(impl))


def _is_package(name: str) -> bool:
    spec = importlib.util.find_spec(name)
    return spec is not None and spec.submodule_search_locations is not None


if not any(isinstance(f, _AliasFinder) for f in sys.meta_path):
    sys.meta_path.insert(0, _AliasFinder())

import cublade_amd as _impl  # noqa: E402  (runs the warm-up)
from cublade_amd import *  # noqa: E402,F401,F403  (the quantization API)
from cublade_amd.bindings.hip import *  # noqa: E402,F401,F403  (binding functions)

_loader = importlib.import_module(__name__ + "._loader")
bindings = importlib.import_module(__name__ + ".bindings")
quantization = importlib.import_module(__name__ + ".quantization")
# Binds the attribute bindings.cuda (importlib sets it on the parent module).
importlib.import_module(__name__ + ".bindings.cuda")

__all__ = [*_impl.__all__]
