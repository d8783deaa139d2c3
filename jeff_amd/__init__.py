"""jeff_amd: the fast path's batched multi-LoRA INT4 linear layer, MI355X-native (HIP kernels for gfx950 behind a
C ABI, PyTorch-ROCm for device memory and streams). See fast_path (Lin, Workspace, lora_add, AdapterPool),
int4_kernels (int4_product), int4 (the kernel weight layout) and product_choice (the product registry)."""
