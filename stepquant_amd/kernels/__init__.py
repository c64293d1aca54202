"""MI355X operators of the packed recurrent-state pool (reference stepquant/kernels).

* ``pool``           PackedStatePool: pages, decode step, encode/decode, slot ops
* ``format_pool``    FormatStatePool: fp32, sym_int*_g128 and dsq_int* baseline pages
* ``writeback``      deferred, graph-captured writer chunks and release windows
* ``resources``      compute-unit-bounded writeback streams
* ``profiles``       writer budgets per captured batch
* ``priority_graph`` decode graph (default priority on this platform)
"""
