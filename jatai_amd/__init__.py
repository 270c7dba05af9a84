"""Jatai INT8 training hot path for MI355X: C-ABI HIP kernels (libjatai.so) behind the reference operator surface."""
