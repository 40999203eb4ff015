// wamx_op_linear_noalloc: wamx_op_linear for callers that cannot allocate
// device memory (code under HIP graph capture, tight serving loops, hosts
// that forbid hipMalloc).  The split-K partials of any product that takes a
// K split (few-token products on the skinny path, and 65..~500-token
// products on small grids, K-sliced 128 x 128 tiles) live in `scratch`, a
// file-scope device array of kScratchBytes that every GPU the library runs on
// holds until the process ends.  Nothing here allocates: no backend is
// created, no workspace is malloc'd; the caller passes its stream, inputs and
// output.  The split is planned as wamx_op_linear plans it with a backend's
// workspace; a product whose partials would then not fit the array is
// refused, so both entry points always take the same slices (same bits).
//
// Every call on a GPU shares that GPU's array and it keeps the last call's
// contents.  The partials are written whole by the part kernel before the
// reduce reads them, so nothing has to start at zero.  Calls that overlap on
// one GPU (two streams, two threads) race on the array: callers serialise
// them, as they serialise a backend.
#include <mutex>

#include "../internal.h"

namespace wamx {

constexpr size_t kScratchBytes = 32ull << 20;   // 32 MiB per GPU
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// Device address of `scratch` on the current device, looked up once per
// device with that device current (each GPU holds its own copy of the array).
static hipError_t scratch_ptr(void ** out) {
    static std::mutex mu;
    static void * ptrs[kMaxDevices] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(mu);
    if (!ptrs[dev]) {
        void * p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        ptrs[dev] = p;
    }
    *out = ptrs[dev];
    return hipSuccess;
}

}  // namespace wamx

using namespace wamx;

extern "C" wamx_status wamx_op_linear_noalloc(void * stream, const void * w, const void * x, int32_t x_type,
                                              const void * bias, int32_t epilogue, const void * residual,
                                              const float * gate, void * y, int64_t M, int64_t N, int64_t K) {
    WAMX_REQUIRE(w && x && y && M > 0 && N > 0 && K > 0, "wamx_op_linear_noalloc: bad arguments");
    WAMX_REQUIRE(x_type == WAMX_TYPE_BF16 || x_type == WAMX_TYPE_F32, "wamx_op_linear_noalloc: x type");
    WAMX_REQUIRE(epilogue >= WAMX_EPI_NONE && epilogue <= WAMX_EPI_BIAS_RESIDUAL, "wamx_op_linear_noalloc: epilogue");
    WAMX_REQUIRE(epilogue == WAMX_EPI_NONE || bias, "wamx_op_linear_noalloc: bias required");
    WAMX_REQUIRE((epilogue != WAMX_EPI_BIAS_GATED && epilogue != WAMX_EPI_BIAS_RESIDUAL) || residual,
                 "wamx_op_linear_noalloc: residual required");
    WAMX_REQUIRE(epilogue != WAMX_EPI_BIAS_GATED || gate, "wamx_op_linear_noalloc: gate required");
    const size_t need = linear_split_bytes(M, N, K, x_type, kBackendWorkspaceBytes);
    WAMX_REQUIRE(need <= kScratchBytes,
                 "wamx_op_linear_noalloc: a %lld x %lld x %lld product needs %zu bytes of split-K scratch, more than "
                 "the %zu this entry point holds; use wamx_op_linear",
                 (long long) N, (long long) M, (long long) K, need, kScratchBytes);
    void * ws = nullptr;
    WAMX_HIP_TRY(scratch_ptr(&ws));
    GemmArgs g;
    g.w = w;
    g.ldw = K;
    g.x = x;
    g.x_type = x_type;
    g.ldx = K;
    g.y = y;
    g.y_type = WAMX_TYPE_BF16;
    g.ldy = M;
    g.M = M;
    g.N = N;
    g.K = K;
    g.epi = epilogue;
    g.bias = bias;
    g.res = residual;
    g.ldres = M;
    g.gate = gate;
    g.ws = ws;
    g.ws_bytes = kScratchBytes;
    WAMX_HIP_TRY(launch_gemm(g, (hipStream_t) stream));
    return WAMX_STATUS_SUCCESS;
}
