"""CPU oracle for the DSA forward -- TEST INFRASTRUCTURE ONLY.

Nothing in the product (the `dsa-cpu-topk_amd` package, libdsa_amd.so and
libdsa_cpu.so) imports, links or runs anything under oracle/.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and only as
the checker or as the timed CPU baseline -- never as the thing measured or
shipped.

  dsa_oracle.py   torch/numpy restatement of the reference forward
  topk_cpu.cpp    C++ restatement of the reference's AVX-512 k-th-largest
                  extension (the timed CPU baseline, kind "port")
  build.py        the build recipe: liboracle_topk.so from topk_cpu.cpp, and
                  oracle/_ref/ from the reference's own topk_avx512.cpp when
                  /root/reference exists
  native.py       ctypes/import loaders for those two builds
"""
