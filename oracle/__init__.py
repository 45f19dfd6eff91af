"""CPU oracle of xenc's Library read — TEST INFRASTRUCTURE ONLY.

A restatement of the reference math in plain PyTorch on the CPU (fp32 in the reference's own
operation order, or fp64 for checking).  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import it, and only as the checker or the timed CPU baseline: the product
package (kv_skill_v2_amd) never imports it and has no CPU path.

Pins (each function is checked by tests/test_oracle.py against something other than itself):
  library_tensors / summaries  closed form S = m/|m| (tests/test_library.py:200-204), centering
                               invariants (:241-261), subset == rebuild (:186-199)
  route                        brute-force rank counting in pure Python, sum/sparsity invariants
                               (tests/test_library.py:126-145)
  boundary_gap                 closed forms: a planted exact tie at the k-th place gives 0, a
                               planted gap gives that gap, k = 0 or k >= C gives +inf
  read                         pure-Python loops on tiny inputs; one-chunk closed form
                               (tests/test_library.py:91-123); linear-read closed form
                               (tests/test_integration.py:139-173); one-hot force_attn
                               (tests/test_d6_force_attn.py:49-63); untied V (test_attn_harvest)
  read_dq                      torch.autograd of the fp64 forward + central finite differences
  selector_weights/apply       sparsity/sum/entropy and matched-norm identity
                               (tests/test_selector.py:25-55)
  decode_read_ref / ref_varlen two-part LSE merge == joint softmax (tests/test_d23_kernels.py:38-48),
                               pure-Python loop restatement on tiny inputs
  select_scores / topk_read    pure-Python loops over heads and slots on tiny inputs; the read
                               over every slot of a one-chunk library == read (the reference's
                               own equivalence, tests/test_topk_read.py:150-170)
  d18_core / d18_lib_read      pure-Python loops per (head, row) on tiny inputs; the routing modes
                               the reference's tests use (tests/test_d18_library.py:73-93); one
                               document == the D13 joint read with absolute RoPE (xenc/d18_library
                               .py:14-15; a planted RoPE-offset mistake moves y by 0.06)
  rms_norm / query / epilogue  closed forms: a constant vector, the output RMS and scale
                               invariance of rms_norm; identity A, the output norm, scale
                               invariance and a pure-Python product for query; gate = 1/2 with
                               B = I, sigmoid(log 3) = 3/4 with gain 2, B = 0 gives exactly 0, and
                               a pure-Python loop for epilogue.  The eps value of rms_norm (1e-6)
                               and the interface's initialisation remain documented parameters:
                               deltaskill, which defines them, is absent.
"""

from .xenc_oracle import *  # noqa: F401,F403
