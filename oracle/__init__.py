"""CPU oracle for the UVU tensor-product convolution.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports this
directory; only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
CPU-baseline leg use it, as the checker (or the timed CPU baseline), never
as the thing measured on the GPU.

Contents (each function cites the reference code it restates):
  wigner.py   real-basis Wigner-3j in e3nn's convention (numpy, fp64)
  sh.py       e3nn real spherical harmonics, l <= 4, component normalisation
  uvu_conv.py dense fp64 restatement of the reference's e3nn oracle:
              TensorProduct on x[src], times env, index_add over dst
"""
