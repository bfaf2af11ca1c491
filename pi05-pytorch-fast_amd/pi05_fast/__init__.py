"""MI355X-native W4A4 prefix-LM GEMM path with the ``pi05_fast.w4a4`` op surface."""

__all__ = ["w4a4"]
