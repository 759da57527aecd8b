"""CPU oracle for the causal attention hot path -- TEST INFRASTRUCTURE ONLY.

Nothing in the product (the HIP library, its C ABI, the C++ launchers or the Python
binding) imports, links or calls anything in this package.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg use it, and only as
the checker (or, for ``cpu_baseline``, as the timed CPU restatement), never as the thing
measured on the GPU.

Contents
--------
attention_ref.py  restatement of the reference's PyTorch attention
                  (pytorch_src/model.py:31-58) in torch-CPU fp32/fp64, its autograd
                  backward, an analytic fp64 backward (numpy) and closed forms.
c_oracle.py       ctypes wrapper of tiled_ref.c, a plain-C restatement of the reference's
                  CUDA kernels (src/kernels/attention.cu): split-transpose, head merge,
                  fused causal softmax fwd/bwd, tiled online-softmax forward with m/l
                  stats, D = rowsum(dO*O), tiled dQ and dK/dV.
gpt_ref.py        restatement of the reference's tiny GPT (pytorch_src/model.py:61-136)
                  with its init recipe (pytorch_src/utils.py:183-209), used to generate
                  the config-1 layer-0 attention fixture.

How each function is pinned (checked against something other than itself) is listed in
the test files ``tests/test_oracle.py`` and ``tests/test_c_oracle.py``:
  * reference known-answer tests (tests/test_kernels.cu:91-120, :210-284);
  * closed forms (V == c => O == c; Q == 0 => prefix means and LSE = ln(i+1); T == 1 =>
    O == V; dO == 0 => zero gradients; V == c => dQ == dK == 0; the KAT's exact dV);
  * fp64 central finite differences of the forward for every gradient;
  * invariants (rows of P sum to 1, rows of dS sum to 0);
  * agreement between independent restatements (torch autograd vs numpy analytic vs C).
The reference's CUDA path cannot be compiled here (no nvcc, no cuBLAS), so there is no
``oracle/_ref`` build.
"""
