"""CPU oracle of the LFM2.5 decode hot path -- TEST INFRASTRUCTURE ONLY.

A plain numpy (+ one C helper) restatement of the reference's CPU PyTorch
BF16 path, used to check the GPU path: only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import it, and never as the thing measured
or shipped. The product path (ryzenai-npu-lab_amd) does not import it.

The arithmetic follows transformers' modeling_lfm2.py (third-party code the
reference calls; pinned by the reference at transformers 5.5.4 + torch 2.8,
docs/setup.md:32) with the per-product rounding of the reference's own
restatement, experiments/006_lfm25_cpu_two_recurrent_layers.py:35-55. Every
function cites the file:line it follows and how it is pinned; see
tests/test_oracle.py. Functions whose BF16 bits only an import of the
third-party library could fix are listed as "parity unpinned" in
lfm25.UNPINNED.
"""
