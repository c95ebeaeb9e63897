"""CPU oracle for Flide's mixture-of-experts layer -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import anything
under `oracle/`, and only as the checker or the timed CPU baseline. The product path (`flide_amd`) never
imports it and raises when its HIP library is missing.

Modules:
  moe_oracle   numpy restatement of flide/kernels/moe.py, fp8.py and the pointwise pieces on the path
  cpu_path     torch-CPU restatement of the reference's eager CPU torch path (transformers' Gemma 4
               router + experts loop), used as the timed CPU baseline

"""
