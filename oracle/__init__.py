"""CPU oracle for the paged-KV decode hot path.

TEST INFRASTRUCTURE ONLY. This package restates the reference's algorithms
on the CPU (numpy in paged_decode.py, C in paged_decode_oracle.c) so the HIP
kernels can be checked against them. Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg may import it, and only to verify results or
as the timed CPU baseline -- never as the product path. The minivllm package
does not import it.

Pinning (see tests/test_oracle_*.py): every function here is checked against
the reference tests' fixtures and tolerances, closed forms (dense softmax,
ctx=1 -> V[0], identical keys -> mean(V)), invariances (block placement,
partition size) and planted mistakes that those checks must reject.
"""
