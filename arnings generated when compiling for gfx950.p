bool hip_ok(kvmem_hip_ctx *ctx, hipError_t e, const char *what) {
