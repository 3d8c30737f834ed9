"""CPU oracle for the batched ragged decode pass — TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the parity checker or the timed CPU
baseline. The product (``chattorrent_amd``) never imports it and has no CPU
fallback.

``oracle.lib`` binds the C restatement of each reference kernel
(``oracle/ccoracle.c``); ``oracle.model`` restates the pass that strings them
together (``web/model/model.js`` blockSegs/forward, ``web/model/stage.js``
#pass) and the page pool (``web/model/model.js`` makePagePool/ensurePages).
"""
