"""CPU oracle for the quantized-linear path — TEST INFRASTRUCTURE, NOT PRODUCT CODE.

A numpy restatement of the reference's algorithms (saransh-debugs/TokenForge,
``tokenforge/kernels/pack.py``, ``reference.py`` and the e4m3 rounding of
``triton/rmsnorm_fp8.py``), used only to check the HIP kernels. Each function cites the
reference lines it follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this package, and only as the checker or the timed CPU baseline. The product package
``tokenforge_amd`` never imports it.

How each part is pinned (tests/unit/test_oracle.py):

* pack / unpack / repack: an independent scalar AutoAWQ packing loop, the sign-bit known
  answer, round trips and element-consistency of the two layouts, brute force on tiny shapes.
* dequant: scalar fp16 arithmetic at group boundaries and zero-point extremes.
* e4m3 encoder: torch's ``.to(torch.float8_e4m3fn)`` (a library routine) on every e4m3 value,
  every midpoint, both neighbours of each midpoint, signed zeros and random values.
* rmsnorm: torch's fp32 ``mean``/``rsqrt`` restatement (reference.py:37-39 as written), which it
  must match except for rare last-ulp differences of the fp32 sum (this oracle sums exactly);
  closed forms for constant rows.
* w4a16 reference: exact rational arithmetic on tiny inputs; IEEE inf/NaN propagation.
* awq_quantize: the reconstruction error bound of the reference's test and scalar re-derivation.
"""
