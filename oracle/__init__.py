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
* ``conv``        -- ConformerConvolution's GLU / causal depthwise conv with the
                     conv cache / LayerNorm / SiLU (parakeet/modules/convolution.py:37-52,107-162)
* ``frontend``    -- log-mel features with dither and the streaming push, 8x
                     convolution subsampling, the pre-encode cache and drop
                     (parakeet/modules/feature_extractor.py, subsample.py;
                     parakeet/engine/model_runner.py:181-252)
* ``rnnt``        -- Predictor / Joiner and the greedy per-frame loop
                     (parakeet/modules/decoder.py:5-86; model_runner.py:347-447)

How each is pinned (the reference ships no tests, fixtures or golden vectors):
see tests/test_oracle_*.py -- closed forms, brute force on tiny inputs, library
special cases (torch SDPA) and invariants.  Nothing here is "parity unpinned".
"""
