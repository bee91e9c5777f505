"""gefen_amd: the Gefen optimizer step, MI355X-native (HIP kernels for gfx950).

``from gefen_amd import Gefen, GefenMuon`` replaces ``from gefen import Gefen, GefenMuon``
(reference __init__.py:1-13); the optimizer classes are loaded lazily.
"""

__all__ = ["Gefen", "GefenMuon", "kernels"]


def __getattr__(name):
    if name == "Gefen":
        from .gefen import Gefen

        return Gefen
    if name == "GefenMuon":
        from .gefen_muon import GefenMuon

        return GefenMuon
    raise AttributeError("module {!r} has no attribute {!r}".format(__name__, name))
