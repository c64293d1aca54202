"""STEPQuant packed-state recurrent update, MI355X-native (gfx950 HIP kernels).

Mirrors the reference package's operator surface: ``stepquant_amd.kernels.pool``,
``stepquant_amd.kernels.format_pool``, ``stepquant_amd.formats``, ``stepquant_amd.packing``,
``stepquant_amd.quantization``, ``stepquant_amd.cli.fingerprint`` and the serving
adapter's pool lifecycle in ``stepquant_amd.sglang.runtime``.
``install_alias()`` registers these modules under the reference's ``stepquant``
names so an adapter written against the reference imports them unchanged.
"""
import importlib
import sys

from .quantization import QuantizationPlan

__all__ = ["QuantizationPlan", "install_alias"]

_ALIASED = ("quantization", "formats", "packing", "cli", "kernels", "kernels.pool", "kernels.writeback",
            "kernels.resources", "kernels.profiles", "kernels.priority_graph", "kernels.format_pool", "sglang",
            "sglang.runtime")


def install_alias(name="stepquant"):
    """Make ``import stepquant.kernels.pool`` (etc.) resolve to this package."""
    sys.modules[name] = sys.modules[__name__]
    for sub in _ALIASED:
        sys.modules[f"{name}.{sub}"] = importlib.import_module(f"{__name__}.{sub}")
    return sys.modules[name]
