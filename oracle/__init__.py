"""CPU oracle for the token-correction path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference algorithm of every function on the hot path, each
module citing the reference file:line it follows. It exists to check the HIP library, never to
stand in for it: only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py`
may import it. The product package `appcorr_amd` does not import it and has no CPU path.

Modules
  bf16     bit-exact bf16 <-> fp32 helpers (round to nearest even)
  plan     top-k selection and the packed query plan            (block.py:358-490)
  rows     gather / scatter / reconstruct+scatter+persist       (token_update.py; block.py:1140-1179)
  nvfp4    NVFP4 quantize / dequantize, bit-exact               (nvfp4_fused.py:53-145)
  model    DINOv3 block: weights, RoPE tables, approx and correct passes
                                                                (block.py:312-349, 942-1191;
                                                                 attention.py:215-278, 393-534)
  pscore   server scores of the approx pass: cls / pseudo-query attention probability and the
           dense / log-sum-exp patch attention probability  (attention.py:241-273;
                                                                 attention_pscore.py:20-98)
  lowp     NVFP4 / FP8 correction linears, scale-and-bias and SwiGLU epilogues
                                                                (fp4_fast_linear.py:103-283;
                                                                 fp8_fast_linear.py:71-196;
                                                                 token_update.py:571-669)
  importance pixel-residual patch scores, image-residual token pruning
                                                                (dinov3_classifier.py:91-197;
                                                                 progressive.py:14-22)

How each function is pinned (the checks live in tests/test_oracle_*.py):
  plan     brute-force ranking on small inputs; torch.topk on distinct scores; KATs (k=0, k=P,
           ties, -inf candidates, NaN)
  rows     numpy fancy indexing identities; byte-equality invariants on unselected rows
  nvfp4    e4m3 rounding against torch's float8_e4m3fn cast; e2m1 against the closed-form grid
           midpoints; hand-derived known-answer blocks; swizzle placement with one distinct scale
           per block; dequantize round-trip error bound and the reference test's rel-L2 < 0.25
  model    LayerNorm / GELU / SDPA against torch.nn.functional; RoPE against the relative-position
           identity of rotations; correction at 100% keep against the full (approx) forward;
           k = 0 gives x + blocks_out_sum exactly
  pscore   torch's own bf16 CPU ops on the same q and K; identical keys give 1/N; a dominant key
           takes the mass; the pseudo query's zero-mean clamp
  lowp     OCP e4m3 known answers through torch's float8_e4m3fn cast; a double-rounding case; every
           x_hat an e2m1 grid value times its block scale; exact GEMMs against float64 products;
           SwiGLU closed forms
  importance the reference's own torch / numpy op sequences; constant-residual closed forms;
           hand-derived pruning plans (min-keep rescue, "an image keeps everything")
Parity of the third-party pieces the reference delegates to (torchao's e2m1 packer nibble order and
NaN handling, Triton's default fp32 divide, torch.topk tie order, cuDNN/cuBLAS accumulation order)
cannot be pinned without running the reference on its hardware: "parity unpinned" for those.
"""
