"""MI355X-native Latent Sparse Attention select+read.

The call surface mirrors the reference's ``lsa_rocm_lab.port`` modules (pipeline,
select_fused, read_kernel_tiled, read_kernel, _tree); every stage runs as a
hand-written HIP kernel for gfx950 in ``_lib/liblsa_rocm.so`` behind a C ABI
(``include/lsa_rocm.h``). There is no CPU fallback: without the library the
entry points raise ``lsa_rocm_lab._abi.ExtensionMissing``.
"""

__version__ = "0.1.0"
