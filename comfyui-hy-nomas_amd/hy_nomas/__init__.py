"""MI355X (gfx950) implementation of Hy-Nomas' quantized DiT linear path.

Modules mirror the reference's interface: `kernels` (activation quantization, block-scaled int8/fp8 GEMM,
fused adaLN + quantization, block_linear), `fused` (adaLN, QK-norm + RoPE, gated residual, PixelUMM QK),
`ops` (int8 g128 weight layout and its Linear), `pixelumm` (fp8 128x128-block weight layout and its Linear)
and `block` (the DiT double-stream block half wired through them).  The kernels live in
libhynomas_hip.so, built from csrc/ by build.py.
"""
