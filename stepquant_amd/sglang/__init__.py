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
"""
