"""CPU oracle of the tiered-cache decode path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg import
this package, and only as the checker (or the timed CPU baseline).  The
product path (kiv_amd) never imports it.

Two restatements of the reference algorithm (Babyhamsta/KIV v0.2.0):

* ``oracle.torch_ref`` -- the reference's op sequence on CPU torch tensors in
  the activation dtype (matmul then ``* scaling`` in the dtype, ``topk``,
  ``unique``, ``amax``, ``gather``, eager softmax attention).  It reproduces
  the reference's dtype rounding; it is also the CPU baseline ("port").
* ``oracle.exact`` -- the same mathematics in float64 numpy (closed forms),
  plus a numpy emulation of the dtype rounding, used to decide which
  selection boundaries are separated enough to compare bit-exactly.

How each part is pinned (none of it is pinned by the reference's own tests,
which check shapes only):
  page summaries       closed form (fp64 mean) and brute force
  coarse/fine scores   closed form q.k*scaling in fp64; dtype emulation
                       checked bit-exactly against torch's own rounding
  selections, union    brute-force sort on small inputs; N=0, N<top_pages,
                       cold<top_p special cases; golden vectors written by
                       the reference itself (tests/golden): torch_ref
                       reproduces them bit for bit, exact ties included
  attention            textbook fp64 softmax attention; P=all losslessness;
                       cold=0 identity; key-permutation invariance
"""
