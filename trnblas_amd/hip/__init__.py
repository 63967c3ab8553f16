"""HIP (gfx950) kernel dispatch of trnblas_amd."""
