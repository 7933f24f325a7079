"""CPU oracle for the selected-attention hot path -- TEST INFRASTRUCTURE ONLY.

A plain restatement (numpy / PyTorch fp32-fp64 on the CPU) of the reference
algorithms, used as the checker by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py.  Nothing in the product imports it; the
product path runs on the HIP kernels of liblsrm_hip.so only.

Modules (each function cites the reference lines it restates):
  pool.py      block mean pooling (torch.segment_reduce mean) under the
               canonical piecewise-sequential fp32 contract
  select.py    per-query-block top-k selection (fp64 scores, forced blocks,
               ties to the lowest block id)
  attention.py selected-block attention forward (o, lse in log2 units) and,
               through torch autograd, backward
  revmap.py    reverse (CSR) query map of a top-k selection
Pins (what checks each function beyond restating it) are listed in each
module's docstring and exercised in tests/test_oracle_*.py.
"""
