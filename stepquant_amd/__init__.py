"""STEPQuant packed-state recurrent update, MI355X-native (gfx950 HIP kernels).

Mirrors the reference package's operator surface: ``stepquant_amd.kernels.pool``,
``stepquant_amd.kernels.format_pool``, ``stepquant_amd.kernels.writeback``,
``stepquant_amd.formats``, ``stepquant_amd.packing``, ``stepquant_amd.quantization``
and ``stepquant_amd.cli.fingerprint``, plus two serving hooks of its own in
``stepquant_amd.sglang``.  ``install_alias()`` binds the reference's
``stepquant.*`` operator modules to these, so the reference's serving adapter
imports them unchanged.
"""
import importlib
import sys

from .quantization import QuantizationPlan

__all__ = ["QuantizationPlan", "install_alias"]

# modules of the reference's operator surface that this package provides
_ALIASED = ("quantization", "formats", "packing", "cli", "kernels", "kernels.pool", "kernels.writeback",
            "kernels.resources", "kernels.profiles", "kernels.priority_graph", "kernels.format_pool",
            "sglang.prefill_reduce")


def install_alias(name="stepquant"):
    """Make ``import stepquant.kernels.pool`` (etc.) resolve to this package.

    When the reference package itself is importable it stays the parent, so
    its serving adapter (``stepquant.sglang``) is used unchanged over these
    modules; otherwise this package stands in for it.  Returns the parent.
    """
    try:
        parent = importlib.import_module(name)
    except ImportError:
        parent = sys.modules[__name__]
        sys.modules[name] = parent
    for sub in _ALIASED:
        module = importlib.import_module(f"{__name__}.{sub}")
        sys.modules[f"{name}.{sub}"] = module
        owner, _, leaf = f"{name}.{sub}".rpartition(".")
        if owner in sys.modules:
            setattr(sys.modules[owner], leaf, module)
    return parent
