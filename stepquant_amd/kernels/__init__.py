"""MI355X operators of the packed recurrent-state pool (reference stepquant/kernels).

* ``pool``           PackedStatePool: pages, decode step, encode/decode, slot ops
* ``writeback``      deferred, graph-captured writer chunks and release windows
* ``resources``      compute-unit-bounded writeback streams
* ``profiles``       writer budgets per captured batch
* ``priority_graph`` decode graph (default priority on this platform)
"""
