"""CPU oracle for Woodcock's per-round speculative-decoding hot path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker -- never as the thing measured or shipped.  The product package
``woodcock_amd`` never imports it and fails loudly when its HIP library is
missing.

Modules
-------
core        ctypes wrapper of ``wc_oracle.c`` (drafter fp32 forward with bf16
            weights, KV compaction, Philox4x64-10 uniforms)
sampling    numpy restatement of python/woodcock/sampling.py and of the
            engine-side distribution handling in python/woodcock/spec.py
greedy      greedy chain/tree verification, tree mask (sampling.py:60-140)
refcpp      ctypes wrapper of ``_ref/libwcref.so`` -- the reference's own C++
            runtime compiled from its sources (built only where the reference
            checkout exists; used to write golden vectors and to cross-check)

Pinning (what checks each function; "parity unpinned" where nothing does)
------------------------------------------------------------------------
core.philox / uniforms     bit-exact vs numpy.random.Philox (library routine)
core.Drafter (fuse/forward/head, fp32)
                           vs the reference C++ Drafter (tests/golden fixtures,
                           tiny config of tests/test_drafter.py:8-21 and a mid
                           config with head_dim 128); restricted head ==
                           gathered full head (tests/test_vocab.py:37-47)
core.kv_compact            known answer of tests/cpp/test_main.cpp:42-50 and
                           the reference KVCache::compact on random patterns
sampling.*                 known answers of tests/test_sampling.py:185-216;
                           chi-square against the exact Markov law with the
                           negative controls of tests/test_sampling.py:36-180;
                           special cases q(x)=0, p==q, T->0
greedy.*                   known answers (test_sampling.py:185-205,
                           test_main.cpp:27-35), reference C++
                           verify_tree_greedy / tree_mask on random trees
bf16 MLX rounding points (nn.Linear, mx.fast.rms_norm/rope/sdpa)
                           parity unpinned (MLX is not available)
"""
