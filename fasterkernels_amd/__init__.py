"""The gfx950 native library behind fskernels' decode hot path.

* ``csrc/fsk_decode.hip`` -- the HIP kernels (split-KV partial and LSE reduce
  kernels for the varlen, paged and dense layouts, the KV write kernel) and
  the C ABI declared in ``include/fsk_decode.h``;
* ``build`` -- compiles ``libfsk_decode.so`` in-tree for gfx950 with hipcc;
* ``native`` -- the ctypes binding of that library (load, status codes,
  workspace sizes, streams);
* ``workloads`` -- the seeded synthetic benchmark configurations.

The Python interface with the reference's module paths is the ``fskernels``
package.
"""
