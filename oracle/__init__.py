"""CPU oracle of the int8 inference path — test infrastructure, never the product.

Imported only by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg. See ``oracle/quant.py`` for the restated arithmetic and what pins each function.
"""
