"""The reference's import surface (ndvbd/Gefen 1.2.3, ``__init__.py:1-13``) over
the MI355X implementation in ``gefen_amd``.

``from gefen import Gefen, GefenMuon`` and the reference's module paths resolve
to this implementation, so code written against the reference runs unchanged:

=================================================  ==========================================
reference module                                   implementation
=================================================  ==========================================
``gefen.gefen``                                    ``gefen_amd.gefen``
``gefen.gefen_muon``                               ``gefen_amd.gefen_muon``
``gefen.partitioning``                             ``gefen_amd.partitioning``
``gefen.quantization``                             ``gefen_amd.quantization``
``gefen.kernels``                                  ``gefen_amd.kernels``
``gefen.kernels.gefen_cuda`` (``load_extension``)  ``gefen_amd.kernels.gefen_hip``
``gefen.kernels.<wrapper>``                        ``gefen_amd.kernels.<wrapper>``
=================================================  ==========================================

Each ``gefen.X`` is the same module object as its implementation (not a copy),
so module-level switches set through either name (``FIND_PERIOD_BACKEND``,
``F_FP32``, ...) are seen by the optimizer.  ``Gefen`` and ``GefenMuon`` load
lazily, as in the reference.
"""

from __future__ import annotations

import importlib
import importlib.abc
import importlib.util
import sys

__all__ = ["Gefen", "GefenMuon", "kernels"]

_ALIASES = {
    "gefen.gefen": "gefen_amd.gefen",
    "gefen.gefen_muon": "gefen_amd.gefen_muon",
    "gefen.partitioning": "gefen_amd.partitioning",
    "gefen.quantization": "gefen_amd.quantization",
    "gefen.kernels": "gefen_amd.kernels",
    "gefen.kernels.gefen_cuda": "gefen_amd.kernels.gefen_hip",
    "gefen.kernels.automatic_gefen_fused": "gefen_amd.kernels.automatic_gefen_fused",
    "gefen.kernels.automatic_vmean": "gefen_amd.kernels.automatic_vmean",
    "gefen.kernels.exact_histogram_fused": "gefen_amd.kernels.exact_histogram_fused",
    "gefen.kernels.period_variance": "gefen_amd.kernels.period_variance",
    "gefen.kernels.lloyd_max_fused": "gefen_amd.kernels.lloyd_max_fused",
}


class _AliasLoader(importlib.abc.MetaPathFinder, importlib.abc.Loader):
    """Finds ``gefen.X`` and hands back the already-imported implementation module."""

    def find_spec(self, fullname, path=None, target=None):
        target_name = _ALIASES.get(fullname)
        if target_name is None:
            return None
        is_pkg = fullname == "gefen.kernels"
        return importlib.util.spec_from_loader(fullname, self, is_package=is_pkg)

    def create_module(self, spec):
        module = importlib.import_module(_ALIASES[spec.name])
        # the import machinery stamps the alias spec on the module it is given;
        # the implementation keeps its own
        self._own_spec = getattr(module, "__spec__", None)
        return module

    def exec_module(self, module):
        own = getattr(self, "_own_spec", None)
        if own is not None:
            module.__spec__ = own


if not any(isinstance(f, _AliasLoader) for f in sys.meta_path):
    sys.meta_path.insert(0, _AliasLoader())


def __getattr__(name):
    if name == "Gefen":
        from .gefen import Gefen

        return Gefen
    if name == "GefenMuon":
        from .gefen_muon import GefenMuon

        return GefenMuon
    if name == "kernels":
        return importlib.import_module("gefen.kernels")
    raise AttributeError("module {!r} has no attribute {!r}".format(__name__, name))
