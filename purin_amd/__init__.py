"""MI355X-native Chambolle--Pock projection (PURIN's CP path) on hand-written HIP kernels."""

__version__ = "0.1.0"
