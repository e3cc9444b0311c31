"""CPU oracle for the verify path -- TEST INFRASTRUCTURE ONLY.

A restatement, in numpy and plain Python, of the reference's algorithms for this path, each
function citing the reference file:line it follows. Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import this package, and only as the checker (or the timed
CPU baseline), never as a compute path of the product: the product runs the HIP kernels of
token-rush_amd/ and raises when they are missing.

Pinning (what checks each function against something other than itself) is listed in the
docstring of each module; a function with no such check says "parity unpinned".
"""
