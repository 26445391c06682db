"""HIP (gfx950) backend modules, one per reference CUDA module:
paged_decode_hip (kernels/cuda/paged_decode_cuda.py), paged_sparse
(kernels/cuda/paged_sparse.py), int8_write (kernels/cuda/int8_write.py)."""
