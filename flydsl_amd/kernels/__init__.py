"""Drop-in launchers for the reference's ``kernels.*`` quantized preshuffle GEMM modules."""
