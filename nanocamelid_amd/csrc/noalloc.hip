// Allocation-free variant of the quantized matmul operator, for callers that cannot allocate
// device memory: code under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc.  The only scratch the matmul needs (the -8 * per-block int8 sums of the
// activations) lives in a file-scope device array instead of context memory.
//
// In host code the array's name is only a host-side handle: its device address is looked up
// once per device (hipGetSymbolAddress, with that device current) when a context is created,
// kept in the context, and only that address is ever passed to kernels.  Every device holds its
// own copy of the array until the process ends.  All calls on one device share it: calls that
// overlap on one device (two streams, or two host threads) race on its contents.  Nothing needs
// to start at zero: the block-sum kernel writes every entry the matmul then reads.
#include "nc_internal.h"

namespace nc {

static __device__ __align__(256) int32_t scratch[kStaticScratchInts];

int static_scratch_address(int32_t** out) {
    void* p = nullptr;
    NC_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    *out = (int32_t*)p;
    return NC_OK;
}

}  // namespace nc

using namespace nc;

extern "C" int nc_matmul_quantized_batch_noalloc(nc_ctx* ctx, const nc_qmat* w, const int8_t* x_i8,
                                                 const float* x_scales, float* out, int batch_size, int64_t rows,
                                                 int64_t cols, void* stream) {
    if (!ctx || !w || !x_i8 || !x_scales || !out)
        return fail(NC_EINVAL, "nc_matmul_quantized_batch_noalloc: null argument");
    if (rows != w->m.rows || cols != w->m.cols)
        return fail(NC_EINVAL, "nc_matmul_quantized_batch_noalloc: shape mismatch");
    if (batch_size < 1 || batch_size > 16)
        return fail(NC_EINVAL, "nc_matmul_quantized_batch_noalloc: batch must be 1..16");
    if ((size_t)batch_size * (size_t)(cols / 32) > kStaticScratchInts)
        return fail(NC_ERANGE, "nc_matmul_quantized_batch_noalloc: batch_size * cols exceeds the static scratch (" +
                                   std::to_string(kStaticScratchInts * 32) + " activation values)");
    if (!ctx->static_scratch) return fail(NC_EINVAL, "nc_matmul_quantized_batch_noalloc: context has no scratch");
    NC_HIP(hipSetDevice(ctx->device));
    hipStream_t st = stream ? (hipStream_t)stream : ctx->stream;
    int rc = launch_block_sums(x_i8, batch_size, (int)cols, ctx->static_scratch, st);
    if (rc) return rc;
    GemmParams p;
    p.kernel = ctx->gemm_kernel;
    p.x = x_i8;
    p.xs = x_scales;
    p.xs8 = ctx->static_scratch;
    p.N = batch_size;
    p.epi = EPI_STORE;
    p.out = out;
    p.ld_out = (int)rows;
    return launch_gemm(w->m, p, st);
}
