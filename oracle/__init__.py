"""CPU oracle for the paged-decode data path -- TEST INFRASTRUCTURE ONLY.

Nothing in ``flashdec_amd`` imports this package.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg use it,
and only as the checker (or, for the baseline, as the timed CPU port) --
never as the thing measured or shipped.

Modules (each function cites the cysong2025/flashdec file:line it restates):

* :mod:`oracle.attention` -- ``paged_decode_attention_ref`` (numpy fp32, the
  reference's per-(sequence, query-head) loop) and a float64 dense brute force.
* :mod:`oracle.rope` -- ``apply_rope`` and the fused RoPE + paged append with
  correctly rounded fp32 transcendentals; bf16/f16 rounding helpers.
* :mod:`oracle.split_policy` -- the vLLM backend's split-count policy.
* :mod:`oracle.torch_loop` -- the same paged decode as fp32 torch-CPU ops in
  the reference's per-(sequence, query-head) loop (bench.py's CPU baseline).

Pinning (how each function is checked before it is trusted) is listed in
``tests/test_oracle.py``; every function here has at least one pin that a
plausible mistake would fail.
"""
