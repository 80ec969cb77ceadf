"""CPU oracle for the GQA attention hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or, for the CPU
baseline, as the reference CPU path that is timed beside the GPU).  The product
path (``breezetoken_amd``) never imports it and has no CPU fallback.

What each function restates, and what pins it (see ``tests/test_oracle.py``):

* ``torch_attention`` / ``torch_attention_einsum`` -- the reference's torch f32
  decode oracle ``_torch_attention`` (breezetoken/backends.py:196-215), SDPA
  branch and einsum fallback branch.  Pinned by: agreement of the two branches,
  f64 brute force, closed forms (S=1, equal keys, dominant key, constant V),
  permutation invariance, the committed config-1 golden vector.
* ``torch_prefill_attention`` / ``torch_prefill_einsum`` -- the causal GQA SDPA
  call of ``_prefill_attn`` (breezetoken/model/prefill.py:56-78) and its
  einsum+tril fallback.  Pinned by: branch agreement, f64 brute force, row i ==
  decode over keys 0..i, row 0 == V[0].
* ``torch_prefill_banded`` -- the explicit-band SDPA of the chunked prefill
  ``Qwen36MoE._attn_batch`` (breezetoken/model/qwen36_moe.py:412-428).  Pinned
  by: pos0 = 0 equals ``torch_prefill_attention``; rows pos0.. of a full
  prefill equal the chunk; f64 brute force with an offset; a top-left-aligned
  mask (``is_causal`` with S < seq) fails it.
* ``split_partition`` / ``split_decode`` / ``combine_lse`` -- the split-KV
  partition, per-split log2-domain LSE + normalised partial, empty-split rule
  and LSE combine of ``gqa_decode`` (breezetoken/kernels/cuda/attention.py:
  104-112, 153-166, 168-189).  Pinned by: combine(split) == unsplit for every
  split count and both partitions, empty split -> (-inf, 0), closed-form LSE.
* ``round_robin_partition`` -- the MI355X kernel's dealing of tiles to splits
  (tile t -> split t % NS), which replaces attention.py:106-112.  Pinned by:
  every token in exactly one split, combine == unsplit.
* ``fixed_decode`` -- the fixed-capacity/device-position contract of
  ``gqa_decode_fixed`` (attention.py:296-301, valid = pos + 1) on top of
  ``torch_attention``.  Pinned by: equality with ``torch_attention`` on the
  prefix, invariance to garbage written past ``pos``.
* ``brute_force_decode_f64`` / ``brute_force_prefill_f64`` -- float64 numpy
  restatements of the attention definition, checked against closed forms.
* ``prep.torch_rms_norm`` / ``prep.torch_rope`` / ``prep.rope_tables`` /
  ``prep.attn_prep`` -- the q/k RMSNorm (breezetoken/backends.py:187-189),
  partial rotate-half RoPE (backends.py:218-226), its cos/sin tables
  (breezetoken/model/layers.py:26-32) and the decode-step preparation of an
  attention layer (layers.py:58-73).  Pinned by (``tests/test_oracle_prep.py``):
  float64 loops in the reference kernel's partner/sign form
  (kernels/cuda/rope.py:31-37) on the reference test's random tables, closed
  forms (constant rows, scale invariance, table angles), rotation properties
  (identity at 0, pair norms, composition), planted mistakes (sum for mean,
  missing weight or eps, flipped sign, interleaved pairs, wrong table row) and
  segment markers for the projection slicing.
* ``gdn.torch_gdn_decode`` -- the Gated DeltaNet one-token step with the f32
  state updated in place (breezetoken/backends.py:242-271).  Pinned by
  (``tests/test_oracle_gdn.py``): a float64 loop written from the update rule,
  closed forms (no write when beta -> -inf, zero state, the delta rule mapping
  kn to v), the h % Hk head grouping, planted mistakes (g without exp, blocked
  grouping, raw beta).
* ``linear.torch_linear`` / ``linear.split_k_linear`` -- the decode matvec
  x.float() @ w.float() (breezetoken/backends.py:182-184), and the same product
  as per-share partial sums added in order (kernels/cuda/gemv.py:18-40 with
  backends.py:327-331), in float64.  Pinned by (``tests/test_oracle_linear.py``):
  float64 products with any number of K shares (split-K invariance), one-hot
  x selecting a row of w, linearity in x, and planted mistakes (transposed w,
  a dropped share).
"""
