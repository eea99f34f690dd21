"""MI355X-native (gfx950) implementation of NERVE's token-sampling stage.

The product is libnerve_sampler.so (C ABI in include/nerve_sampler.h, HIP
kernels in csrc/); `sampler` is its Python front end and `workloads` builds
the seeded synthetic inputs of the benchmark configurations.
"""
