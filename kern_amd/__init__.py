"""kern_amd — MI355X-native implementation of kern's MXFP4 matmul path.

Hand-written gfx950 kernels (kern_amd/csrc/kern_mx.hip) behind a C ABI (include/kern_amd.h,
kern_amd/lib/libkern_amd.so); `kern_amd.ops` mirrors the manifest ops over it, `kern_amd.workload`
draws the seeded synthetic inputs. Submodules are imported explicitly (`from kern_amd import ops`).
"""
