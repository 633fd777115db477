"""CPU oracle for the continuous-batching data path -- TEST INFRASTRUCTURE ONLY.

Plain numpy restatements of the reference algorithms (Anant3133/memforge), each
function citing the reference file:line it follows. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this package, and only as the checker / the timed CPU baseline: the
product path (``memforge_amd``) never imports, links or calls it.

Modules
  paging     slot mapping, KV write/gather, write index, ragged pack
  attention  paged / varlen attention (fp64 brute force and the fp32
             block-wise online-softmax form)
  rejection  speculative rejection sampling with explicit randomness
  bf16       torch's float32 -> bfloat16 rounding, restated on bit patterns

Each function's parity pin (what it was checked against) is listed in
``tests/test_oracle.py``; none of them is "parity unpinned".
"""
