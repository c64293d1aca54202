"""Serving hooks this build adds to the reference's SGLang adapter.

The reference adapter (stepquant/sglang: plan artifacts, pool lifecycle,
decode hooks, graph capture) runs unchanged over this package's pools once
``stepquant_amd.install_alias()`` binds its ``stepquant.*`` operator modules
here.  Two hooks are this build's own:

* ``extend.kernel_extend`` runs the chunked prefill straight from and into
  the pages (``PackedStatePool.extend``) instead of the reference's decode,
  upstream chunk kernel and encode round trip;
* ``prefill_reduce.forward`` / ``all_reduce`` keep the reference's contract
  (tensor-parallel prefill sums accumulated in fp32) for the module name the
  adapter's plugin registers.

The reference plugin's ``verify_hooks`` (sglang/plugin.py:5-11) only counts
hooks defined in its own ``stepquant.sglang.*`` modules, so it would not
notice these two failing to patch; ``verify_hooks`` here counts both.
"""

# modules whose hooks must all be patched before serving starts: the
# reference adapter's (sglang/plugin.py:8) and this package's
_HOOK_MODULES = ("stepquant.sglang.runtime", "stepquant.sglang.admission", "stepquant.sglang.logits",
                 "stepquant.sglang.prefill_reduce", "stepquant_amd.sglang.extend",
                 "stepquant_amd.sglang.prefill_reduce")


def verify_hooks(registry=None):
    """Raise ``RuntimeError`` unless every registered STEPQuant hook -- the
    reference adapter's and this package's -- has been patched.

    ``registry`` is SGLang's ``HookRegistry`` (imported when omitted): its
    ``_hooks`` maps a target to ``(type, fn, ...)`` entries and ``_patched``
    holds the targets already patched.
    """
    if registry is None:
        from sglang.srt.plugins.hook_registry import HookRegistry as registry
    required = [target for target, hooks in registry._hooks.items()
                if any(getattr(entry[1], "__module__", "") in _HOOK_MODULES for entry in hooks)]
    missing = set(required) - set(registry._patched)
    if not required or missing:
        raise RuntimeError(f"STEPQuant plugin hooks incomplete: {sorted(missing)}; refusing FP32 fallback")
    return sorted(required)
