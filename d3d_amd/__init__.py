"""d3d_amd: MI355X (gfx950) kernels for D3D's per-step speculative hot path.

Public surface mirrors the reference's call sites:

* ``d3d_amd.speculative_sampling`` -- ``verify_speculative_block``,
  ``verify_speculative_block_sparse``, ``SpeculativeSampleResult`` plus the
  batched ``accept_fused`` / ``greedy_accept``.
"""
__version__ = "0.1.0"
