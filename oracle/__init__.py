"""CPU oracle for the AMASS decode-time sparse-attention hot path -- TEST INFRASTRUCTURE.

A numpy restatement of the reference algorithm (Js-Hwang1/amass-kv, src/amass/...), used
only as the checker: by tests/, by ``__graft_entry__.smoke()`` and by the cpu_baseline leg
of bench.py.  The product path (amass-kv_amd/amass, libamass_hip.so) never imports it and
has no CPU fallback.

Modules and what pins each function (beyond "it restates the reference"):

  quant.py   q_limbs (quad_score_cuda.py:902-935)      pinned: 128*hi+lo == qi, |qi-q/qs|<=.5
             quant/pack_i4 (build.py:297-348)           pinned: round trip, int4 nibble layout
  score.py   quad_score (quad_score.py:35-107)          pinned: closed form from raw keys
                                                        (s q.mu + s^2/2P |dc q|^2 at full rank),
                                                        eigen-sign invariance
             quad_comb / r8_comb (exact int64 sums)     pinned: brute force Python ints
             nrm_combine (quad_score.py:276-315)        pinned: hand-computed small case
             r8_score (score.py:30-120)                 pinned: = logsumexp of the true page
                                                        logits when the page rank <= r
             clse_score (quad_score.py:156-276)         pinned: == r8_score at resid 0; iso
                                                        term on a hand-built page; nrm/max
  select.py  derive (select.py:30-45)                   pinned: config-0 known answer b=13
             topb (select.py:60-101 + tie rule)         pinned: sorted() brute force
             nucleus (build spec; bridge :117-133)      pinned: minimality brute force
             exp_det / f2u                              pinned: |exp_det/np.exp-1| < 4 ulp,
                                                        f2u order-preserving
  decode.py  attend (decode.py:128-241 math)            pinned: dense softmax attention
             split_merge (decode.py:146-153, merge.py:21-50)  pinned: split invariance
  build.py   page_factors (build.py:396-412, quad_build.py:124-198)
                                                        pinned: exact reconstruction at
                                                        rank <= r, sig2 == svd(dc)^2,
                                                        Vk orthonormal, rank-1 page by hand
             quad_summary / r8_summary (quant rules)    pinned: via quant + the factors
             clse_summary (quad_build.py:38-54)         pinned: resid == energy beyond the
                                                        top r' singular values
  tier.py    plan (residency.py:45-139)                 pinned: hand-worked LRU example,
                                                        page2slot/slot2page inverse,
                                                        victims are the oldest untouched
  stage.py   invalidate (residency.py:251-278)          pinned: hand-worked example
             begin_step (staging.py:87-232,312-343)     pinned: hand-worked two steps;
             scatter (staging.py:51-80)                 simulations: every written token's
                                                        V reads back (I1), free stack is a
                                                        partition (I3), shared block,
                                                        small flush list, exhaustion

The reference ships no tests, fixtures or golden vectors for this path (its own tests
directory is absent), so every check above is a closed form, an invariant or a brute
force; tests/golden/ holds small fixtures this oracle generated, frozen so that later
changes to the oracle itself are caught.
"""
