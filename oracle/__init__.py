"""Oracle: CPU restatement of odunola499/parakeet-streaming's paged-KV hot path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker or the timed CPU baseline -- never as the product path.  The product
(``parakeet-streaming_amd/parakeet_amd``) never imports it and has no CPU
fallback.

Modules (each function cites the reference file:line it restates):

* ``dense_cache`` -- dense shift-buffer ModelCache (parakeet/modules/cache.py)
* ``paging``      -- FIFO page pool + ring block table model, page append/gather
* ``masks``       -- _create_streaming_masks loop (parakeet/modules/encoder.py:167-227)
* ``relpos``      -- sinusoid table, pos slice, rel_shift (parakeet/modules/attention.py:23-83)
* ``attention``   -- ConformerAttention core (parakeet/modules/attention.py:85-125)
* ``dense_path``  -- torch-CPU fp32 dense encoder-attention step (the CPU baseline)

How each is pinned (the reference ships no tests, fixtures or golden vectors):
see tests/test_oracle_*.py -- closed forms, brute force on tiny inputs, library
special cases (torch SDPA) and invariants.  Nothing here is "parity unpinned".
"""
