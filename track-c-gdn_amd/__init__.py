"""MI355X-native (gfx950) Gated DeltaNet decode and prefill operators.

The directory name is not a Python identifier, so the package is imported
under the module name ``track_c_gdn_amd`` by a path loader (see
``load_package`` in ``__graft_entry__.py``), or its entry files
``gdn_decode_qk4_v8_d128_k_last/kernel.py`` and
``gdn_prefill_qk4_v8_d128_k_last/kernel.py`` are loaded by path, as a
FlashInfer-Bench style harness does with ``kernel.py::run``.

Submodules:
  decode   -- decode ``run`` / ``run_dps`` / ``gdn_decode`` / ``decode_pool_``
  prefill  -- prefill ``run`` / ``run_dps`` / ``gdn_prefill`` (fused or split path)
  conv     -- the short causal conv1d + SiLU ahead of GDN (q/k/v straight to GDN layout)
  backward -- prefill backward from the per-chunk states, gate gradients, autograd operator
  inputs   -- seeded synthetic workloads
  build    -- hipcc recipe for libgdn_hip.so
  _capi    -- ctypes binding of include/gdn_hip.h
"""

__all__ = ["decode", "prefill", "conv", "backward", "inputs", "build"]
