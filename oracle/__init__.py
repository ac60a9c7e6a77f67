"""CPU restatement of the reference's scoring-and-selection path.

THIS PACKAGE IS TEST INFRASTRUCTURE. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker or as the timed
CPU baseline, never as part of the product path (``retrieve_amd`` never imports it).

Every function cites the reference file:line it restates. Paths are relative to the
reference checkout (``rmnigm/retrieve``). What pins each function (golden vectors, known-answer
tests, closed forms, brute force) is listed in each module's docstring; a function with no such
check says "parity unpinned" there.

Modules:
- ``quantize``  per-row int8 quantization, SimHash sign packing (``indexing/quantize.py``).
- ``select``    exact top-k with ties to the lower index, the two-list merge
                (``evaluation/bench/oracle.py:83-92``, ``fork_search_cuda.cu:65-81``).
- ``scan``      int8 / Hamming / dense brute-force scans + top-k (``ops/reference/*``).
- ``filters``   exact clause predicate, MurmurHash3 token hash, Bloom bundle layout and plan
                evaluation (``functional.py:173-185``, ``bloom_index_util.cuh:60-222``,
                ``bloom_indexer.cpp:27-114``, ``bloom_index_search_cuda.cu:305-613``).
- ``baseline``  the reference's CPU path (chunked ``mm`` + top-k merge) timed by ``bench.py``.
"""
