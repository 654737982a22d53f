// C-ABI entry points (declared in include/wmma_ops_amd.h).
//
// Each entry point validates every argument first -- shapes, pointers, leading
// dimensions, alignment, workspace -- and only then enqueues kernels on the caller's
// stream.  Nothing here allocates or synchronises.  Errors are reported as a status
// code plus a per-thread message (wmma_last_error).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

#include "kernels.hpp"
#include "plan.hpp"

using namespace wmma_amd;

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int ok() {
    g_last_error.clear();
    return WMMA_OK;
}

int hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return ok();
    return fail(WMMA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

constexpr int kMaxDevices = 64;
int g_cu_count[kMaxDevices];
std::once_flag g_cu_once[kMaxDevices];

int current_cus() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    return wmma_device_cu_count(dev);
}

// Largest byte offset a buffer-resource load may use (offsets are 32-bit, and
// 0x80000000 and above mark masked lanes).
constexpr int64_t kMaxOffset = 0x7fffffffLL;

size_t round256(size_t x) { return (x + 255) & ~(size_t)255; }

// Workspace bytes, behind the split-K partial sums, for zero-padded dense copies of the
// operands whose rows break 16-byte vectors: A [M][K8] when `a`, B [K][N8] when `b` (K8, N8
// rounded up to 8), each copy 256-byte aligned (256 bytes of slack align the first).
size_t repack_bytes(int M, int N, int K, bool a, bool b) {
    if ((!a && !b) || M <= 0 || N <= 0 || K <= 0) return 0;
    const size_t K8 = ((size_t)K + 7) & ~(size_t)7, N8 = ((size_t)N + 7) & ~(size_t)7;
    return 256 + (a ? round256((size_t)M * K8 * 2) : 0) + (b ? round256((size_t)K * N8 * 2) : 0);
}

}  // namespace

// Scratch of the allocation-free GEMM entry point (wmma_gemm_f16f32_noalloc): the split-K
// partial sums live in this file-scope device array instead of a caller workspace.  Each
// GPU the library runs on holds its own copy, at its own address, until the process ends.
// In host code `scratch` names a host-side stand-in, never the device memory: the device
// address is fetched once per device with hipGetSymbolAddress and only that is used.
constexpr size_t kScratchBytes = size_t(32) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
void* g_scratch_ptr[kMaxDevices];
hipError_t g_scratch_rc[kMaxDevices];
std::once_flag g_scratch_once[kMaxDevices];
// Cross-stream ordering of the calls that use a device's scratch array: each such call
// (outside stream capture) first makes its stream wait for the event the previous call
// recorded after its own launches, when that call ran on another stream.  The event is
// created by the first such call on the device made outside capture; later calls create
// nothing.  g_scratch_mu serialises host threads around wait + launch + record.
hipEvent_t g_scratch_ev[kMaxDevices];
bool g_scratch_ev_made[kMaxDevices];
hipStream_t g_scratch_last[kMaxDevices];
bool g_scratch_recorded[kMaxDevices];
std::mutex g_scratch_mu[kMaxDevices];

// Device address of `scratch` on the current device (once per device, with it current).
int scratch_for_current_device(void** out, int* dev_out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return fail(WMMA_ERR_UNSUPPORTED, "device index %d", dev);
    std::call_once(g_scratch_once[dev], [dev] {
        void* ptr = nullptr;
        g_scratch_rc[dev] = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        g_scratch_ptr[dev] = g_scratch_rc[dev] == hipSuccess ? ptr : nullptr;
    });
    if (g_scratch_rc[dev] != hipSuccess) return hip_status(g_scratch_rc[dev], "hipGetSymbolAddress(scratch)");
    *out = g_scratch_ptr[dev];
    *dev_out = dev;
    return WMMA_OK;
}

// Before a call's launches on `st` (with g_scratch_mu[dev] held): wait for the previous
// scratch user when it ran on another stream.  *ordered is false under stream capture,
// where no event is waited on or recorded (a captured graph is ordered by whoever
// launches it).
int scratch_order_before(int dev, hipStream_t st, bool* ordered) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(st, &cs);
    if (e != hipSuccess) return hip_status(e, "hipStreamIsCapturing");
    *ordered = cs == hipStreamCaptureStatusNone;
    if (*ordered && !g_scratch_ev_made[dev]) {
        e = hipEventCreateWithFlags(&g_scratch_ev[dev], hipEventDisableTiming);
        if (e != hipSuccess) return hip_status(e, "hipEventCreate(scratch)");
        g_scratch_ev_made[dev] = true;
    }
    if (*ordered && g_scratch_recorded[dev] && g_scratch_last[dev] != st) {
        e = hipStreamWaitEvent(st, g_scratch_ev[dev], 0);
        if (e != hipSuccess) return hip_status(e, "hipStreamWaitEvent(scratch)");
    }
    return WMMA_OK;
}

// After the launches: the next scratch user on another stream waits for this point.
int scratch_order_after(int dev, hipStream_t st) {
    hipError_t e = hipEventRecord(g_scratch_ev[dev], st);
    if (e != hipSuccess) return hip_status(e, "hipEventRecord(scratch)");
    g_scratch_last[dev] = st;
    g_scratch_recorded[dev] = true;
    return WMMA_OK;
}
}  // namespace

extern "C" {

const char* wmma_last_error(void) { return g_last_error.c_str(); }

int wmma_abi_version(void) { return WMMA_OPS_AMD_ABI_VERSION; }

int wmma_device_cu_count(int device) {
    if (device < 0 || device >= kMaxDevices) return 256;
    std::call_once(g_cu_once[device], [device] {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
            n <= 0)
            n = 256;
        g_cu_count[device] = n;
    });
    return g_cu_count[device];
}

int wmma_gemm_plan_make(int M, int N, int K, int tile_cfg, int num_cus, wmma_gemm_plan* out) {
    if (!out) return fail(WMMA_ERR_INVALID_ARG, "plan output pointer is NULL");
    if (M < 0 || N < 0 || K < 0) return fail(WMMA_ERR_INVALID_ARG, "negative GEMM dimension");
    if (tile_cfg < WMMA_TILE_AUTO || tile_cfg >= WMMA_TILE_COUNT)
        return fail(WMMA_ERR_INVALID_ARG,
                    "Invalid tile_config: 0=64x64, 1=128x64, 2=256x64, 3=128x128, 4=256x128, "
                    "5=256x256");
    int rc = make_plan(M, N, K, tile_cfg, num_cus, out);
    return rc == WMMA_OK ? ok() : fail(rc, "planner rejected the shape");
}

int wmma_gemm_plan_make_within(int M, int N, int K, int tile_cfg, int num_cus,
                               size_t max_workspace_bytes, wmma_gemm_plan* out) {
    if (!out) return fail(WMMA_ERR_INVALID_ARG, "plan output pointer is NULL");
    if (M < 0 || N < 0 || K < 0) return fail(WMMA_ERR_INVALID_ARG, "negative GEMM dimension");
    if (tile_cfg < WMMA_TILE_AUTO || tile_cfg >= WMMA_TILE_COUNT)
        return fail(WMMA_ERR_INVALID_ARG,
                    "Invalid tile_config: 0=64x64, 1=128x64, 2=256x64, 3=128x128, 4=256x128, "
                    "5=256x256");
    int rc = make_plan_within(M, N, K, tile_cfg, num_cus, max_workspace_bytes, out);
    return rc == WMMA_OK ? ok() : fail(rc, "planner rejected the shape");
}

size_t wmma_gemm_workspace_size(int M, int N, int K, int tile_cfg) {
    wmma_gemm_plan p{};
    if (make_plan(M, N, K, tile_cfg, current_cus(), &p) != WMMA_OK) return 0;
    // Contiguous operands (lda = K, ldb = N, 16-byte aligned) break 16-byte rows exactly
    // when K or N is not a multiple of 8; the skinny kernel reads such a B in place.
    return p.workspace_bytes +
           repack_bytes(M, N, K, K % 8 != 0, N % 8 != 0 && p.kernel != WMMA_KERNEL_SKINNY);
}

// Shared checks and launch of wmma_gemm_f16f32 / wmma_gemm_f16f32_plan /
// wmma_gemm_f16f32_noalloc.  `plan` is NULL for the planner's own plan (tile_cfg), else an
// explicit plan for exactly this shape.  use_scratch: the split-K partials go to the
// library's own scratch array (the caller passes no workspace).
static int gemm_run(const void* A, int64_t lda, const void* B, int64_t ldb, const float* C_in,
                    int64_t ldc_in, float* C_out, int64_t ldc, int M, int N, int K, float alpha,
                    float beta, int tile_cfg, const wmma_gemm_plan* explicit_plan,
                    void* workspace, size_t workspace_bytes, void* stream,
                    bool use_scratch = false) {
    if (M < 0 || N < 0 || K < 0) return fail(WMMA_ERR_INVALID_ARG, "negative GEMM dimension");
    if (tile_cfg < WMMA_TILE_AUTO || tile_cfg >= WMMA_TILE_COUNT)
        return fail(WMMA_ERR_INVALID_ARG,
                    "Invalid tile_config: 0=64x64, 1=128x64, 2=256x64, 3=128x128, 4=256x128, "
                    "5=256x256");
    if (M == 0 || N == 0) return ok();  // empty output
    if (!C_out) return fail(WMMA_ERR_INVALID_ARG, "C_out is NULL");
    if (ldc < N) return fail(WMMA_ERR_INVALID_ARG, "ldc (%lld) < N (%d)", (long long)ldc, N);
    const bool use_c = beta != 0.0f && C_in != nullptr;
    if (use_c && ldc_in < N)
        return fail(WMMA_ERR_INVALID_ARG, "ldc_in (%lld) < N (%d)", (long long)ldc_in, N);
    if (K > 0) {
        if (!A || !B) return fail(WMMA_ERR_INVALID_ARG, "A or B is NULL");
        if (lda < K) return fail(WMMA_ERR_INVALID_ARG, "lda (%lld) < K (%d)", (long long)lda, K);
        if (ldb < N) return fail(WMMA_ERR_INVALID_ARG, "ldb (%lld) < N (%d)", (long long)ldb, N);
        // 32-bit buffer offsets: one 256-row A tile and one 64-row B stage must fit (also
        // with the leading dimensions of repacked copies, at most 7 elements longer).
        if ((256 + 1) * (lda + 7) * 2 > kMaxOffset || (64 + 1) * (ldb + 7) * 2 > kMaxOffset ||
            (int64_t)kSkinnyMaxMWide * (lda + 7) * 2 > kMaxOffset)
            return fail(WMMA_ERR_UNSUPPORTED, "leading dimension too large for 32-bit offsets");
    }
    // The allocation-free entry point plans within its scratch array.
    const size_t plan_cap = use_scratch ? kScratchBytes : SIZE_MAX;
    wmma_gemm_plan plan{};
    if (explicit_plan) {
        // Rebuild the plan from its choices for this shape: a plan made for another shape,
        // or edited by hand, is rejected rather than launched.  A two-part plan is the
        // planner's own for this shape or nothing.
        int rc = explicit_plan->edge_dim != WMMA_EDGE_NONE
                     ? make_plan(M, N, K, WMMA_TILE_AUTO, current_cus(), &plan)
                     : make_custom_plan(M, N, K, explicit_plan->kernel, explicit_plan->tile_cfg,
                                        explicit_plan->split_k, &plan);
        if (rc != WMMA_OK || plan.kernel != explicit_plan->kernel ||
            plan.k_per_split != explicit_plan->k_per_split ||
            plan.split_k != explicit_plan->split_k ||
            plan.workspace_bytes != explicit_plan->workspace_bytes ||
            plan.edge_dim != explicit_plan->edge_dim || plan.edge_at != explicit_plan->edge_at ||
            (plan.kernel == WMMA_KERNEL_TILED && plan.tile_cfg != explicit_plan->tile_cfg))
            return fail(WMMA_ERR_INVALID_ARG, "plan does not describe this shape (make it with "
                                              "wmma_gemm_plan_custom or wmma_gemm_plan_make)");
    } else {
        int rc = make_plan_within(M, N, K, tile_cfg, current_cus(), plan_cap, &plan);
        if (rc != WMMA_OK) return fail(rc, "planner rejected the shape");
    }
    int scratch_dev = -1;
    bool scratch_ordered = false;
    std::unique_lock<std::mutex> scratch_lock;
    if (use_scratch && plan.workspace_bytes > 0) {
        if (plan.workspace_bytes > kScratchBytes)
            return fail(WMMA_ERR_WORKSPACE,
                        "split-K needs %zu bytes of scratch; the allocation-free entry point "
                        "holds at most %zu (use wmma_gemm_f16f32 with a workspace)",
                        plan.workspace_bytes, kScratchBytes);
        if (int rc = scratch_for_current_device(&workspace, &scratch_dev)) return rc;
        workspace_bytes = kScratchBytes;
        scratch_lock = std::unique_lock<std::mutex>(g_scratch_mu[scratch_dev]);
        if (int rc = scratch_order_before(scratch_dev, static_cast<hipStream_t>(stream),
                                          &scratch_ordered))
            return rc;
    }
    if (plan.workspace_bytes > 0) {
        if (!workspace)
            return fail(WMMA_ERR_WORKSPACE, "split-K needs a workspace of %zu bytes",
                        plan.workspace_bytes);
        if (workspace_bytes < plan.workspace_bytes)
            return fail(WMMA_ERR_WORKSPACE, "workspace too small: %zu < %zu bytes", workspace_bytes,
                        plan.workspace_bytes);
        if ((reinterpret_cast<uintptr_t>(workspace) & 3u) != 0)
            return fail(WMMA_ERR_MISALIGNED, "workspace must be 4-byte aligned");
    }
    // An operand whose rows break 16-byte vectors (K or N not a multiple of 8, a leading
    // dimension that is not, or an address off 16 bytes) is copied into a zero-padded dense
    // buffer behind the partial sums when the workspace holds it, and the vector kernels
    // run on the copy; without that room (or from the allocation-free entry point) the
    // element-wise kernels read it in place.  The skinny kernel streams B once, so there a
    // 4-byte-aligned B is read in place by dword-aligned 16-byte loads instead (a copy
    // would triple its traffic).  The padding is zero and every kernel masks rows and
    // columns at M, N and K, so the result is the same either way.
    bool a_vec = K % 8 == 0 && lda % 8 == 0 && aligned16(A);
    bool b_vec = N % 8 == 0 && ldb % 8 == 0 && aligned16(B);
    const bool skinny = plan.kernel == WMMA_KERNEL_SKINNY;
    const bool b_al4 = (reinterpret_cast<uintptr_t>(B) & 3u) == 0;
    const bool b_copy = !b_vec && !(skinny && b_al4);
    if (K > 0 && (!a_vec || b_copy) && !use_scratch && workspace &&
        workspace_bytes >= plan.workspace_bytes + repack_bytes(M, N, K, !a_vec, b_copy)) {
        const hipStream_t st = static_cast<hipStream_t>(stream);
        unsigned char* dst = reinterpret_cast<unsigned char*>(
            round256(reinterpret_cast<uintptr_t>(workspace) + plan.workspace_bytes));
        if (!a_vec) {
            const int64_t K8 = ((int64_t)K + 7) & ~(int64_t)7;
            if (int rc = hip_status(launch_gemm_repack(A, lda, M, K, dst, st), "gemm repack A"))
                return rc;
            A = dst;
            lda = K8;
            a_vec = true;
            dst += round256((size_t)M * (size_t)K8 * 2);
        }
        if (b_copy) {
            const int64_t N8 = ((int64_t)N + 7) & ~(int64_t)7;
            if (int rc = hip_status(launch_gemm_repack(B, ldb, K, N, dst, st), "gemm repack B"))
                return rc;
            B = dst;
            ldb = N8;
            b_vec = true;
        }
    }
    const bool vec = K > 0 && a_vec && b_vec;
    // One launch of plan `pl` on the sub-GEMM whose output starts at row r0, column c0.
    auto launch_part = [&](const wmma_gemm_plan& pl, int r0, int c0, int Mp, int Np) {
        GemmLaunch g{};
        g.A = static_cast<const uint16_t*>(A) + (int64_t)r0 * lda;
        g.B = static_cast<const uint16_t*>(B) + c0;
        g.C_in = use_c ? C_in + (int64_t)r0 * ldc_in + c0 : nullptr;
        g.C_out = C_out + (int64_t)r0 * ldc + c0;
        g.workspace = workspace;
        g.lda = lda;
        g.ldb = ldb;
        g.ldc_in = ldc_in;
        g.ldc = ldc;
        g.M = Mp;
        g.N = Np;
        g.K = K;
        g.alpha = alpha;
        g.beta = beta;
        g.vec = vec;
        g.skinny_b = pl.kernel == WMMA_KERNEL_SKINNY && !vec && K > 0 && a_vec && b_al4
                         ? (ldb % 2 == 0 ? 2 : 3)
                         : 0;
        g.plan = pl;
        return hip_status(launch_gemm(g, static_cast<hipStream_t>(stream)), "gemm launch");
    };
    auto launch_all = [&]() -> int {
        if (plan.edge_dim == WMMA_EDGE_NONE) return launch_part(plan, 0, 0, M, N);
        // Two parts, one after the other on the stream (the edge's split-K partial sums
        // reuse the workspace): the bulk on whole waves of 256x256 tiles, then the edge with
        // the plan the planner gives its own shape.  Column offsets keep 16-byte alignment
        // (edge_at is a multiple of 256) and 4-byte alignment of B for the skinny kernel.
        const bool rows = plan.edge_dim == WMMA_EDGE_ROWS;
        const int at = plan.edge_at;
        wmma_gemm_plan edge{};
        if (make_plan_within(rows ? M - at : M, rows ? N : N - at, K, WMMA_TILE_AUTO,
                             current_cus(), plan_cap, &edge) != WMMA_OK ||
            edge.edge_dim != WMMA_EDGE_NONE || edge.workspace_bytes > plan.workspace_bytes)
            return fail(WMMA_ERR_INVALID_ARG, "inconsistent two-part plan");
        if (int rc = launch_part(plan, 0, 0, rows ? at : M, rows ? N : at)) return rc;
        return rows ? launch_part(edge, at, 0, M - at, N) : launch_part(edge, 0, at, M, N - at);
    };
    const int rc = launch_all();
    if (scratch_dev >= 0 && scratch_ordered) {
        const int rc2 = scratch_order_after(scratch_dev, static_cast<hipStream_t>(stream));
        if (rc == WMMA_OK) return rc2;
    }
    return rc;
}

int wmma_gemm_f16f32(const void* A, int64_t lda, const void* B, int64_t ldb, const float* C_in,
                     int64_t ldc_in, float* C_out, int64_t ldc, int M, int N, int K, float alpha,
                     float beta, int tile_cfg, void* workspace, size_t workspace_bytes,
                     void* stream) {
    return gemm_run(A, lda, B, ldb, C_in, ldc_in, C_out, ldc, M, N, K, alpha, beta, tile_cfg,
                    nullptr, workspace, workspace_bytes, stream);
}

int wmma_gemm_f16f32_noalloc(const void* A, int64_t lda, const void* B, int64_t ldb,
                             const float* C_in, int64_t ldc_in, float* C_out, int64_t ldc, int M,
                             int N, int K, float alpha, float beta, int tile_cfg, void* stream) {
    return gemm_run(A, lda, B, ldb, C_in, ldc_in, C_out, ldc, M, N, K, alpha, beta, tile_cfg,
                    nullptr, nullptr, 0, stream, /*use_scratch=*/true);
}

size_t wmma_gemm_noalloc_scratch_bytes(void) { return kScratchBytes; }

int wmma_gemm_plan_custom(int M, int N, int K, int kernel, int tile_cfg, int split_k,
                          wmma_gemm_plan* out) {
    if (!out) return fail(WMMA_ERR_INVALID_ARG, "NULL plan");
    if (make_custom_plan(M, N, K, kernel, tile_cfg, split_k, out) != WMMA_OK)
        return fail(WMMA_ERR_INVALID_ARG,
                    "no such plan: kernel %d, tile %d, split %d for M=%d N=%d K=%d", kernel,
                    tile_cfg, split_k, M, N, K);
    return ok();
}

int wmma_gemm_f16f32_plan(const void* A, int64_t lda, const void* B, int64_t ldb,
                          const float* C_in, int64_t ldc_in, float* C_out, int64_t ldc, int M,
                          int N, int K, float alpha, float beta, const wmma_gemm_plan* plan,
                          void* workspace, size_t workspace_bytes, void* stream) {
    if (!plan) return fail(WMMA_ERR_INVALID_ARG, "NULL plan");
    return gemm_run(A, lda, B, ldb, C_in, ldc_in, C_out, ldc, M, N, K, alpha, beta,
                    WMMA_TILE_AUTO, plan, workspace, workspace_bytes, stream);
}

// ------------------------------------------------------------------------------ INT4 --
static int check_int4_shape(int K, int N) {
    if (K <= 0 || N <= 0) return fail(WMMA_ERR_INVALID_ARG, "K and N must be positive");
    if (K % 64 != 0) return fail(WMMA_ERR_UNSUPPORTED, "K (%d) must be a multiple of 64", K);
    if (N % 32 != 0) return fail(WMMA_ERR_UNSUPPORTED, "N (%d) must be a multiple of 32", N);
    return WMMA_OK;
}

int wmma_int4_prepack(const int32_t* qweight, int K, int N, int32_t* packed, void* stream) {
    if (int rc = check_int4_shape(K, N)) return rc;
    if (!qweight || !packed) return fail(WMMA_ERR_INVALID_ARG, "NULL pointer");
    if (!aligned16(packed)) return fail(WMMA_ERR_MISALIGNED, "packed output must be 16-byte aligned");
    if ((reinterpret_cast<uintptr_t>(qweight) & 3u) != 0)
        return fail(WMMA_ERR_MISALIGNED, "qweight must be 4-byte aligned");
    return hip_status(launch_int4_prepack(qweight, K, N, packed, static_cast<hipStream_t>(stream)),
                      "int4 prepack launch");
}

int wmma_int4_unprepack(const int32_t* packed, int K, int N, int32_t* qweight, void* stream) {
    if (int rc = check_int4_shape(K, N)) return rc;
    if (!qweight || !packed) return fail(WMMA_ERR_INVALID_ARG, "NULL pointer");
    if (!aligned16(packed)) return fail(WMMA_ERR_MISALIGNED, "packed input must be 16-byte aligned");
    if ((reinterpret_cast<uintptr_t>(qweight) & 3u) != 0)
        return fail(WMMA_ERR_MISALIGNED, "qweight must be 4-byte aligned");
    return hip_status(
        launch_int4_unprepack(packed, K, N, qweight, static_cast<hipStream_t>(stream)),
        "int4 unprepack launch");
}

int wmma_int4_unpack(const int32_t* qweight, int K, int N, uint8_t* q, void* stream) {
    if (K <= 0 || N <= 0 || K % 8 != 0)
        return fail(WMMA_ERR_INVALID_ARG, "K must be a positive multiple of 8 and N positive");
    if (!qweight || !q) return fail(WMMA_ERR_INVALID_ARG, "NULL pointer");
    if ((reinterpret_cast<uintptr_t>(qweight) & 3u) != 0)
        return fail(WMMA_ERR_MISALIGNED, "qweight must be 4-byte aligned");
    return hip_status(launch_int4_unpack(qweight, K, N, q, static_cast<hipStream_t>(stream)),
                      "int4 unpack launch");
}

int wmma_int4_prepack_params(const void* scales, const void* zeros, int zeros_format, int K,
                             int N, int group_size, void* scales_out, int32_t* zeros_out,
                             void* stream) {
    if (int rc = check_int4_shape(K, N)) return rc;
    if (group_size <= 0 || K % group_size != 0)
        return fail(WMMA_ERR_INVALID_ARG, "group_size (%d) must divide K (%d)", group_size, K);
    if (zeros_format != WMMA_ZEROS_PACKED && zeros_format != WMMA_ZEROS_U8)
        return fail(WMMA_ERR_INVALID_ARG, "zeros format %d cannot be sliced", zeros_format);
    if (!scales || !zeros || !scales_out || !zeros_out) return fail(WMMA_ERR_INVALID_ARG, "NULL pointer");
    if ((reinterpret_cast<uintptr_t>(scales) & 1u) != 0 ||
        (reinterpret_cast<uintptr_t>(scales_out) & 1u) != 0)
        return fail(WMMA_ERR_MISALIGNED, "scales must be 2-byte aligned");
    if ((zeros_format == WMMA_ZEROS_PACKED && (reinterpret_cast<uintptr_t>(zeros) & 3u) != 0) ||
        (reinterpret_cast<uintptr_t>(zeros_out) & 3u) != 0)
        return fail(WMMA_ERR_MISALIGNED, "packed zeros must be 4-byte aligned");
    return hip_status(launch_int4_params_slice(scales, zeros, zeros_format, K / group_size, N,
                                               scales_out, zeros_out,
                                               static_cast<hipStream_t>(stream)),
                      "int4 params launch");
}

// Fused decode layout: G % 128 == 0 with G / 128 a power of two (a 128-deep K step never
// straddles two groups), K % 128 == 0.
static bool fused_group_ok(int K, int G) {
    return G > 0 && G % 128 == 0 && ((G / 128) & (G / 128 - 1)) == 0 && K % G == 0;
}

size_t wmma_int4_fused_bytes(int K, int N) {
    if (K <= 0 || N <= 0 || K % 128 != 0 || N % 32 != 0) return 0;
    return (size_t)(N / 16) * (size_t)fused_slice_bytes(K);
}

int wmma_int4_prepack_fused(const int32_t* qweight, const void* scales, const void* zeros,
                            int zeros_format, int K, int N, int group_size, int32_t* fused,
                            void* stream) {
    if (int rc = check_int4_shape(K, N)) return rc;
    if (K % 128 != 0) return fail(WMMA_ERR_UNSUPPORTED, "K (%d) must be a multiple of 128", K);
    if (!fused_group_ok(K, group_size))
        return fail(WMMA_ERR_UNSUPPORTED,
                    "group_size (%d) must be 128 * 2^j and divide K (%d) for the fused layout",
                    group_size, K);
    if (zeros_format != WMMA_ZEROS_PACKED && zeros_format != WMMA_ZEROS_U8)
        return fail(WMMA_ERR_INVALID_ARG, "zeros format %d cannot be fused", zeros_format);
    if (!qweight || !scales || !zeros || !fused) return fail(WMMA_ERR_INVALID_ARG, "NULL pointer");
    if (!aligned16(fused)) return fail(WMMA_ERR_MISALIGNED, "fused output must be 16-byte aligned");
    if ((reinterpret_cast<uintptr_t>(qweight) & 3u) != 0)
        return fail(WMMA_ERR_MISALIGNED, "qweight must be 4-byte aligned");
    if ((reinterpret_cast<uintptr_t>(scales) & 1u) != 0)
        return fail(WMMA_ERR_MISALIGNED, "scales must be 2-byte aligned");
    if (zeros_format == WMMA_ZEROS_PACKED && (reinterpret_cast<uintptr_t>(zeros) & 3u) != 0)
        return fail(WMMA_ERR_MISALIGNED, "packed zeros must be 4-byte aligned");
    return hip_status(launch_int4_prepack_fused(qweight, scales, zeros, zeros_format, K, N,
                                                group_size, fused, static_cast<hipStream_t>(stream)),
                      "int4 fused prepack launch");
}

int wmma_int4_unprepack_fused(const int32_t* fused, int K, int N, int group_size,
                              int32_t* qweight, void* scales, int32_t* zeros, void* stream) {
    if (int rc = check_int4_shape(K, N)) return rc;
    if (K % 128 != 0) return fail(WMMA_ERR_UNSUPPORTED, "K (%d) must be a multiple of 128", K);
    if (!fused_group_ok(K, group_size))
        return fail(WMMA_ERR_UNSUPPORTED,
                    "group_size (%d) must be 128 * 2^j and divide K (%d) for the fused layout",
                    group_size, K);
    if (!qweight || !scales || !zeros || !fused) return fail(WMMA_ERR_INVALID_ARG, "NULL pointer");
    if (!aligned16(fused)) return fail(WMMA_ERR_MISALIGNED, "fused input must be 16-byte aligned");
    if ((reinterpret_cast<uintptr_t>(qweight) & 3u) != 0 ||
        (reinterpret_cast<uintptr_t>(zeros) & 3u) != 0)
        return fail(WMMA_ERR_MISALIGNED, "qweight and zeros must be 4-byte aligned");
    if ((reinterpret_cast<uintptr_t>(scales) & 1u) != 0)
        return fail(WMMA_ERR_MISALIGNED, "scales must be 2-byte aligned");
    return hip_status(launch_int4_unprepack_fused(fused, K, N, group_size, qweight, scales, zeros,
                                                  static_cast<hipStream_t>(stream)),
                      "int4 fused unprepack launch");
}

size_t wmma_w4a16_workspace_size(int M, int N, int K, int group_size) {
    if (M <= 0 || N <= 0 || K <= 0 || K % 64 != 0 || group_size <= 0) return 0;
    // The plan depends on operand alignment only through the choice of the matrix-pipe
    // decode kernel; report the larger of the two possible workspaces.
    size_t need = 0;
    for (bool aligned : {true, false}) {
        const W4A16Plan pl = w4a16_plan(M, N, K, group_size, current_cus(), aligned);
        if (pl.split > 1) need = std::max(need, (size_t)pl.split * M * N * sizeof(float));
    }
    return need;
}

int wmma_w4a16_plan_make(int M, int N, int K, int group_size, int num_cus, wmma_w4a16_plan* out) {
    if (!out) return fail(WMMA_ERR_INVALID_ARG, "NULL plan");
    if (M <= 0 || N <= 0 || K <= 0 || K % 64 != 0 || N % 32 != 0 || group_size <= 0 ||
        group_size % 32 != 0 || K % group_size != 0)
        return fail(WMMA_ERR_INVALID_ARG, "invalid W4A16 shape M=%d N=%d K=%d G=%d", M, N, K,
                    group_size);
    const W4A16Plan pl = w4a16_plan(M, N, K, group_size, num_cus > 0 ? num_cus : current_cus(), true);
    out->kernel = pl.kind;
    out->split_k = pl.split;
    out->k_per_split = pl.k_per_split;
    out->workspace_bytes = pl.split > 1 ? (size_t)pl.split * M * N * sizeof(float) : 0;
    return ok();
}

static int w4a16_run(const void* A, int64_t lda, const int32_t* packed, const void* scales,
                     const void* zeros, int zeros_format, int M, int N, int K, int group_size,
                     void* Y, int64_t ldy, bool y_half, void* workspace, size_t workspace_bytes,
                     void* stream) {
    if (M < 0) return fail(WMMA_ERR_INVALID_ARG, "M must be non-negative");
    if (int rc = check_int4_shape(K, N)) return rc;
    if (group_size <= 0 || group_size % 32 != 0 || K % group_size != 0)
        return fail(WMMA_ERR_UNSUPPORTED,
                    "group_size (%d) must be a positive multiple of 32 dividing K (%d)", group_size,
                    K);
    if (zeros_format != WMMA_ZEROS_PACKED && zeros_format != WMMA_ZEROS_U8 &&
        zeros_format != WMMA_ZEROS_SLICED && zeros_format != WMMA_W4_FUSED)
        return fail(WMMA_ERR_INVALID_ARG, "unknown zeros format %d", zeros_format);
    const bool fused = zeros_format == WMMA_W4_FUSED;
    if (fused) {
        if (K % 128 != 0 || !fused_group_ok(K, group_size))
            return fail(WMMA_ERR_UNSUPPORTED,
                        "the fused layout needs K %% 128 == 0 and group_size = 128 * 2^j "
                        "(K=%d, group_size=%d)", K, group_size);
        if (!w4a16_fused_decode_ok(M, K))
            return fail(WMMA_ERR_UNSUPPORTED,
                        "the fused layout is read by the decode kernel only (M <= 4; M=%d, K=%d)",
                        M, K);
    }
    if (M == 0) return ok();
    if (!A || !packed || !Y || (!fused && (!scales || !zeros)))
        return fail(WMMA_ERR_INVALID_ARG, "NULL pointer");
    if (lda < K || ldy < N) return fail(WMMA_ERR_INVALID_ARG, "leading dimension too small");
    if (!aligned16(A) || lda % 8 != 0)
        return fail(WMMA_ERR_MISALIGNED, "A must be 16-byte aligned with lda a multiple of 8");
    if (!aligned16(packed)) return fail(WMMA_ERR_MISALIGNED, "packed weights must be 16-byte aligned");
    if (!fused && (reinterpret_cast<uintptr_t>(scales) & 1u) != 0)
        return fail(WMMA_ERR_MISALIGNED, "scales must be 2-byte aligned");
    if (!fused && zeros_format != WMMA_ZEROS_U8 && (reinterpret_cast<uintptr_t>(zeros) & 3u) != 0)
        return fail(WMMA_ERR_MISALIGNED, "packed zeros must be 4-byte aligned");
    // 32-bit buffer offsets: the tiled kernels address A from their first row (at most 256
    // rows), the LDS-DMA GEMM its weights from its first 32-column tile (at most 8 tiles of
    // K * 16 bytes), and every kernel the group parameters from their start.
    if ((int64_t)std::min(M, 256) * lda * 2 > kMaxOffset)
        return fail(WMMA_ERR_UNSUPPORTED, "activation rows too long for 32-bit offsets");
    if ((int64_t)8 * K * 16 > kMaxOffset)
        return fail(WMMA_ERR_UNSUPPORTED, "K (%d) too large for 32-bit weight offsets", K);
    if ((int64_t)(K / group_size) * N * 2 > kMaxOffset)
        return fail(WMMA_ERR_UNSUPPORTED, "group parameters too large for 32-bit offsets");
    W4A16Launch w{};
    const bool aligned = (reinterpret_cast<uintptr_t>(scales) & 7u) == 0 &&
                         (zeros_format != WMMA_ZEROS_U8 ||
                          (reinterpret_cast<uintptr_t>(zeros) & 3u) == 0);
    if (fused) {
        w.plan.kind = W4_DECODE_MFMA;
        w.plan.split = 1;
        w.plan.k_per_split = K;
    } else {
        w.plan = w4a16_plan(M, N, K, group_size, current_cus(), aligned);
    }
    const size_t need = w.plan.split > 1 ? (size_t)w.plan.split * M * N * sizeof(float) : 0;
    if (need > 0 && (!workspace || workspace_bytes < need))
        return fail(WMMA_ERR_WORKSPACE, "W4A16 split-K needs a workspace of %zu bytes", need);
    w.A = A;
    w.lda = lda;
    w.packed = packed;
    w.scales = scales;
    w.zeros = zeros;
    w.zeros_format = zeros_format;
    w.M = M;
    w.N = N;
    w.K = K;
    w.G = group_size;
    w.Y = static_cast<float*>(Y);
    w.y_half = y_half;
    w.ldy = ldy;
    w.workspace = workspace;
    return hip_status(launch_w4a16(w, static_cast<hipStream_t>(stream)), "w4a16 launch");
}

int wmma_w4a16_gemm(const void* A, int64_t lda, const int32_t* packed, const void* scales,
                    const void* zeros, int zeros_format, int M, int N, int K, int group_size,
                    float* Y, int64_t ldy, void* workspace, size_t workspace_bytes, void* stream) {
    return w4a16_run(A, lda, packed, scales, zeros, zeros_format, M, N, K, group_size, Y, ldy,
                     false, workspace, workspace_bytes, stream);
}

int wmma_w4a16_gemm_f16out(const void* A, int64_t lda, const int32_t* packed,
                           const void* scales, const void* zeros, int zeros_format, int M, int N,
                           int K, int group_size, void* Y, int64_t ldy, void* workspace,
                           size_t workspace_bytes, void* stream) {
    if (Y && (reinterpret_cast<uintptr_t>(Y) & 1u) != 0)
        return fail(WMMA_ERR_MISALIGNED, "fp16 Y must be 2-byte aligned");
    return w4a16_run(A, lda, packed, scales, zeros, zeros_format, M, N, K, group_size, Y, ldy,
                     true, workspace, workspace_bytes, stream);
}

int wmma_int4_from_awq(const int32_t* qweight_awq, const int32_t* qzeros_awq, int K, int N,
                       int group_size, int32_t* qweight, int32_t* zeros, void* stream) {
    if (K <= 0 || N <= 0 || K % 8 != 0 || N % 8 != 0)
        return fail(WMMA_ERR_INVALID_ARG, "K and N must be positive multiples of 8");
    if (group_size <= 0 || K % group_size != 0)
        return fail(WMMA_ERR_INVALID_ARG, "group_size (%d) must divide K (%d)", group_size, K);
    if (!qweight_awq || !qzeros_awq || !qweight || !zeros)
        return fail(WMMA_ERR_INVALID_ARG, "NULL pointer");
    for (const void* ptr : {(const void*)qweight_awq, (const void*)qzeros_awq, (const void*)qweight,
                            (const void*)zeros})
        if ((reinterpret_cast<uintptr_t>(ptr) & 3u) != 0)
            return fail(WMMA_ERR_MISALIGNED, "int32 tensors must be 4-byte aligned");
    return hip_status(launch_int4_from_awq(qweight_awq, qzeros_awq, K, N, K / group_size, qweight,
                                           zeros, static_cast<hipStream_t>(stream)),
                      "awq conversion launch");
}

int wmma_int4_from_gptq_zeros(const int32_t* qzeros, int K, int N, int group_size,
                              int zero_format, int32_t* zeros, int32_t* overflow, void* stream) {
    if (K <= 0 || N <= 0 || N % 8 != 0)
        return fail(WMMA_ERR_INVALID_ARG, "K must be positive and N a positive multiple of 8");
    if (group_size <= 0 || K % group_size != 0)
        return fail(WMMA_ERR_INVALID_ARG, "group_size (%d) must divide K (%d)", group_size, K);
    if (zero_format != WMMA_GPTQ_V1 && zero_format != WMMA_GPTQ_V2)
        return fail(WMMA_ERR_INVALID_ARG, "unknown GPTQ zero format %d", zero_format);
    if (!qzeros || !zeros) return fail(WMMA_ERR_INVALID_ARG, "NULL pointer");
    for (const void* ptr : {(const void*)qzeros, (const void*)zeros, (const void*)overflow})
        if ((reinterpret_cast<uintptr_t>(ptr) & 3u) != 0)
            return fail(WMMA_ERR_MISALIGNED, "int32 tensors must be 4-byte aligned");
    return hip_status(launch_int4_gptq_zeros(qzeros, K / group_size, N,
                                             zero_format == WMMA_GPTQ_V1 ? 1 : 0, zeros, overflow,
                                             static_cast<hipStream_t>(stream)),
                      "gptq zeros launch");
}

int wmma_int4_permute_rows(const int32_t* qweight, const int32_t* perm, int K, int N,
                           int32_t* qweight_out, void* stream) {
    if (K <= 0 || N <= 0 || K % 8 != 0)
        return fail(WMMA_ERR_INVALID_ARG, "K must be a positive multiple of 8 and N positive");
    if (!qweight || !perm || !qweight_out) return fail(WMMA_ERR_INVALID_ARG, "NULL pointer");
    if (qweight == qweight_out) return fail(WMMA_ERR_INVALID_ARG, "the permutation cannot run in place");
    for (const void* ptr : {(const void*)qweight, (const void*)perm, (const void*)qweight_out})
        if ((reinterpret_cast<uintptr_t>(ptr) & 3u) != 0)
            return fail(WMMA_ERR_MISALIGNED, "int32 tensors must be 4-byte aligned");
    return hip_status(launch_int4_permute_rows(qweight, perm, K, N, qweight_out,
                                               static_cast<hipStream_t>(stream)),
                      "row permutation launch");
}

// ----------------------------------------------------------------------------- flash --
namespace {

// Head dims the kernels take: multiples of 8 (16-byte rows) from 8 to 256.
constexpr int kFlashMaxDFwd = 256, kFlashMaxDBwd = 256;
int flash_head_dim_check(int D, int max_d) {
    if (D < 8 || D > max_d || D % 8 != 0)
        return fail(WMMA_ERR_UNSUPPORTED, "head_dim %d (supported: multiples of 8 from 8 to %d)", D,
                    max_d);
    return WMMA_OK;
}

// Shape checks shared by the dense forward and backward entry points.
int flash_dense_check(int B, int H, int Hkv, int Sq, int Sk, int D, float scale, int max_d) {
    if (B < 0 || H < 0 || Sq < 0 || Sk < 0) return fail(WMMA_ERR_INVALID_ARG, "negative dimension");
    if (int rc = flash_head_dim_check(D, max_d)) return rc;
    if (!(scale > 0.0f) || !std::isfinite(scale))
        return fail(WMMA_ERR_INVALID_ARG, "scale must be positive and finite");
    if (H > 0 && (Hkv <= 0 || H % Hkv != 0))
        return fail(WMMA_ERR_INVALID_ARG, "key/value heads (%d) must divide query heads (%d)", Hkv, H);
    if ((int64_t)Sq * D * 2 > kMaxOffset || (int64_t)Sk * D * 2 > kMaxOffset)
        return fail(WMMA_ERR_UNSUPPORTED, "sequence too long for 32-bit offsets");
    if ((int64_t)B * H > 2147483647LL) return fail(WMMA_ERR_UNSUPPORTED, "too many heads");
    return WMMA_OK;
}

int flash_varlen_check(int B, int H, int Hkv, int total_q, int total_k, int max_q, int max_k,
                       int D, float scale, int max_d) {
    if (B < 0 || H < 0 || total_q < 0 || total_k < 0 || max_q < 0 || max_k < 0)
        return fail(WMMA_ERR_INVALID_ARG, "negative dimension");
    if (int rc = flash_head_dim_check(D, max_d)) return rc;
    if (!(scale > 0.0f) || !std::isfinite(scale))
        return fail(WMMA_ERR_INVALID_ARG, "scale must be positive and finite");
    if (H > 0 && (Hkv <= 0 || H % Hkv != 0))
        return fail(WMMA_ERR_INVALID_ARG, "key/value heads (%d) must divide query heads (%d)", Hkv, H);
    // 32-bit offsets inside one sequence of one head
    if ((int64_t)max_q * H * D * 2 > kMaxOffset || (int64_t)max_k * Hkv * D * 2 > kMaxOffset)
        return fail(WMMA_ERR_UNSUPPORTED, "sequence too long for 32-bit offsets");
    if ((int64_t)B * H > 2147483647LL) return fail(WMMA_ERR_UNSUPPORTED, "too many heads");
    return WMMA_OK;
}

bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }

}  // namespace

// Grouped-query attention without a causal mask, dense layout: the H/Hkv query heads of a
// group are consecutive rows of Q, O and lse and attend to the same keys, so they run as one
// sequence of (H/Hkv) Sq rows against their key/value head -- every query row computes
// exactly as before, and each K/V tile is read once per group instead of once per query
// head (for decoding, H/Hkv times fewer bytes).  A causal mask depends on the row's position
// in its own head's sequence, so causal shapes keep one sequence per query head.
static void flash_pack_groups(int causal, int* H, int Hkv, int* Sq) {
    if (causal || Hkv <= 0 || *H <= Hkv || (int64_t)*Sq * (*H / Hkv) > INT32_MAX) return;
    *Sq *= *H / Hkv;
    *H = Hkv;
}

// Dense forward; `workspace` (may be NULL) enables the key-range split when it holds the
// split's partial sums.
static int flash_fwd_run(const void* Q, const void* K, const void* V, void* O, float* lse, int B,
                         int H, int Hkv, int Sq, int Sk, int D, float scale, int causal,
                         void* workspace, size_t workspace_bytes, void* stream) {
    if (int rc = flash_dense_check(B, H, Hkv, Sq, Sk, D, scale, kFlashMaxDFwd)) return rc;
    if (B == 0 || H == 0 || Sq == 0) return ok();
    if (Sk == 0) return fail(WMMA_ERR_INVALID_ARG, "Sk must be positive when Sq > 0");
    if (!Q || !K || !V || !O) return fail(WMMA_ERR_INVALID_ARG, "NULL pointer");
    if (!aligned16(Q) || !aligned16(K) || !aligned16(V) || !aligned16(O))
        return fail(WMMA_ERR_MISALIGNED, "Q, K, V and O must be 16-byte aligned");
    if (lse && !aligned4(lse)) return fail(WMMA_ERR_MISALIGNED, "lse must be 4-byte aligned");
    FlashLaunch f{};
    f.Q = Q;
    f.K = K;
    f.V = V;
    f.O = O;
    f.B = B;
    f.H = H;
    f.Hkv = Hkv;
    f.Sq = Sq;
    f.Sk = Sk;
    f.D = D;
    f.scale = scale;
    f.causal = causal != 0;
    f.lse = lse;
    flash_pack_groups(causal, &f.H, f.Hkv, &f.Sq);
    if (workspace) {
        const int split = flash_kv_split(B, f.H, Hkv, f.Sq, Sk, D, current_cus());
        const size_t need = flash_fwd_workspace_bytes(B, f.H, f.Sq, Sk, D, split);
        if (split > 1 && workspace_bytes >= need) {
            if (!aligned16(workspace))
                return fail(WMMA_ERR_MISALIGNED, "workspace must be 16-byte aligned");
            f.kv_split = split;
            f.workspace = workspace;
        }
    }
    return hip_status(launch_flash_fwd(f, static_cast<hipStream_t>(stream)), "flash launch");
}

int wmma_flash_attn_fwd_lse(const void* Q, const void* K, const void* V, void* O, float* lse,
                            int B, int H, int Hkv, int Sq, int Sk, int D, float scale, int causal,
                            void* stream) {
    return flash_fwd_run(Q, K, V, O, lse, B, H, Hkv, Sq, Sk, D, scale, causal, nullptr, 0, stream);
}

size_t wmma_flash_attn_fwd_workspace_size(int B, int H, int Hkv, int Sq, int Sk, int D,
                                          int causal) {
    if (B <= 0 || H <= 0 || Hkv <= 0 || H % Hkv != 0 || Sq <= 0 || Sk <= 0 || D <= 0 ||
        D % 8 != 0 || D > kFlashMaxDFwd)
        return 0;
    flash_pack_groups(causal, &H, Hkv, &Sq);
    return flash_fwd_workspace_bytes(B, H, Sq, Sk, D,
                                     flash_kv_split(B, H, Hkv, Sq, Sk, D, current_cus()));
}

int wmma_flash_attn_fwd_ws(const void* Q, const void* K, const void* V, void* O, float* lse,
                           int B, int H, int Hkv, int Sq, int Sk, int D, float scale, int causal,
                           void* workspace, size_t workspace_bytes, void* stream) {
    return flash_fwd_run(Q, K, V, O, lse, B, H, Hkv, Sq, Sk, D, scale, causal, workspace,
                         workspace_bytes, stream);
}

int wmma_flash_attn_fwd_gqa(const void* Q, const void* K, const void* V, void* O, int B, int H,
                            int Hkv, int Sq, int Sk, int D, float scale, int causal, void* stream) {
    return wmma_flash_attn_fwd_lse(Q, K, V, O, nullptr, B, H, Hkv, Sq, Sk, D, scale, causal, stream);
}

int wmma_flash_attn_varlen_fwd_lse(const void* Q, const void* K, const void* V, void* O,
                                   float* lse, const int32_t* cu_seqlens_q,
                                   const int32_t* cu_seqlens_k, int B, int H, int Hkv,
                                   int total_q, int total_k, int max_seqlen_q, int max_seqlen_k,
                                   int D, float scale, int causal, void* stream) {
    if (int rc = flash_varlen_check(B, H, Hkv, total_q, total_k, max_seqlen_q, max_seqlen_k, D,
                                    scale, kFlashMaxDFwd))
        return rc;
    if (B == 0 || H == 0 || total_q == 0 || max_seqlen_q == 0) return ok();
    if (!Q || !K || !V || !O || !cu_seqlens_q || !cu_seqlens_k)
        return fail(WMMA_ERR_INVALID_ARG, "NULL pointer");
    if (!aligned16(Q) || !aligned16(K) || !aligned16(V) || !aligned16(O))
        return fail(WMMA_ERR_MISALIGNED, "Q, K, V and O must be 16-byte aligned");
    if (!aligned4(cu_seqlens_q) || !aligned4(cu_seqlens_k))
        return fail(WMMA_ERR_MISALIGNED, "cu_seqlens must be 4-byte aligned");
    if (lse && !aligned4(lse)) return fail(WMMA_ERR_MISALIGNED, "lse must be 4-byte aligned");
    FlashLaunch f{};
    f.Q = Q;
    f.K = K;
    f.V = V;
    f.O = O;
    f.B = B;
    f.H = H;
    f.Hkv = Hkv;
    f.Sq = max_seqlen_q;
    f.Sk = max_seqlen_k;
    f.D = D;
    f.scale = scale;
    f.causal = causal != 0;
    f.cu_q = cu_seqlens_q;
    f.cu_k = cu_seqlens_k;
    f.total_q = total_q;
    f.total_k = total_k;
    f.lse = lse;
    return hip_status(launch_flash_fwd(f, static_cast<hipStream_t>(stream)), "flash launch");
}

int wmma_flash_attn_varlen_fwd(const void* Q, const void* K, const void* V, void* O,
                               const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int B,
                               int H, int Hkv, int total_q, int total_k, int max_seqlen_q,
                               int max_seqlen_k, int D, float scale, int causal, void* stream) {
    return wmma_flash_attn_varlen_fwd_lse(Q, K, V, O, nullptr, cu_seqlens_q, cu_seqlens_k, B, H,
                                          Hkv, total_q, total_k, max_seqlen_q, max_seqlen_k, D,
                                          scale, causal, stream);
}

int wmma_flash_attn_fwd(const void* Q, const void* K, const void* V, void* O, int B, int H,
                        int Sq, int Sk, int D, float scale, int causal, void* stream) {
    return wmma_flash_attn_fwd_gqa(Q, K, V, O, B, H, H, Sq, Sk, D, scale, causal, stream);
}

size_t wmma_flash_attn_bwd_workspace_size(int B, int H, int Sq) {
    if (B <= 0 || H <= 0 || Sq <= 0) return 0;
    return (size_t)2 * sizeof(float) * (size_t)B * (size_t)H * (size_t)Sq;
}

namespace {
int flash_bwd_run(FlashBwdLaunch& f, void* workspace, size_t workspace_bytes, void* stream) {
    // Query-side tensors are read only when there are query rows, key-side ones only when
    // there are key rows (either side may be empty).
    const int64_t rows = flash_bwd_workspace_rows(f);
    const bool has_q = rows > 0, has_k = f.cu_k ? f.total_k > 0 : (int64_t)f.B * f.Hkv * f.Sk > 0;
    if ((has_q && (!f.dO || !f.Q || !f.O || !f.lse || !f.dQ)) || (has_k && (!f.K || !f.V || !f.dK || !f.dV)))
        return fail(WMMA_ERR_INVALID_ARG, "NULL pointer");
    if (!aligned16(f.dO) || !aligned16(f.Q) || !aligned16(f.K) || !aligned16(f.V) ||
        !aligned16(f.O) || !aligned16(f.dQ) || !aligned16(f.dK) || !aligned16(f.dV))
        return fail(WMMA_ERR_MISALIGNED, "dO, Q, K, V, O, dQ, dK and dV must be 16-byte aligned");
    if (!aligned4(f.lse)) return fail(WMMA_ERR_MISALIGNED, "lse must be 4-byte aligned");
    const size_t need = (size_t)2 * sizeof(float) * (size_t)rows;
    if (need > 0) {
        if (!workspace) return fail(WMMA_ERR_WORKSPACE, "NULL workspace");
        if (!aligned4(workspace)) return fail(WMMA_ERR_MISALIGNED, "workspace must be 4-byte aligned");
        if (workspace_bytes < need)
            return fail(WMMA_ERR_WORKSPACE, "workspace of %zu bytes, %zu needed", workspace_bytes, need);
    }
    f.ws = static_cast<float*>(workspace);
    // Dense grouped-query attention whose dK/dV workgroups would leave most CUs idle: the
    // group's query heads are split over more workgroups when the workspace also holds their
    // fp32 partial dK, dV (behind the row statistics, 256-byte aligned).
    if (!f.cu_q && has_q && has_k) {
        const int gs =
            flash_bwd_group_split(f.B, f.H, f.Hkv, f.Sq, f.Sk, f.D, f.causal, current_cus());
        const size_t part = flash_bwd_split_bytes(f.B, f.Hkv, f.Sk, f.D, gs);
        if (gs > 1 && workspace_bytes >= round256(need) + part && aligned16(workspace)) {
            f.gsplit = gs;
            f.kv_part = reinterpret_cast<float*>(static_cast<unsigned char*>(workspace) + round256(need));
        }
    }
    return hip_status(launch_flash_bwd(f, static_cast<hipStream_t>(stream)), "flash backward launch");
}
}  // namespace

size_t wmma_flash_attn_bwd_split_workspace_size(int B, int H, int Hkv, int Sq, int Sk, int D,
                                                int causal) {
    if (B <= 0 || H <= 0 || Hkv <= 0 || H % Hkv != 0 || Sq <= 0 || Sk <= 0 || D <= 0 ||
        D % 8 != 0 || D > kFlashMaxDBwd)
        return wmma_flash_attn_bwd_workspace_size(B, H, Sq);
    const size_t need = wmma_flash_attn_bwd_workspace_size(B, H, Sq);
    const int gs = flash_bwd_group_split(B, H, Hkv, Sq, Sk, D, causal != 0, current_cus());
    return gs > 1 ? round256(need) + flash_bwd_split_bytes(B, Hkv, Sk, D, gs) : need;
}

int wmma_flash_attn_bwd(const void* dO, const void* Q, const void* K, const void* V, const void* O,
                        const float* lse, void* dQ, void* dK, void* dV, void* workspace,
                        size_t workspace_bytes, int B, int H, int Hkv, int Sq, int Sk, int D,
                        float scale, int causal, void* stream) {
    if (int rc = flash_dense_check(B, H, Hkv, Sq, Sk, D, scale, kFlashMaxDBwd)) return rc;
    if (B == 0 || H == 0 || (Sq == 0 && Sk == 0)) return ok();
    if (Sk == 0) return fail(WMMA_ERR_INVALID_ARG, "Sk must be positive when Sq > 0");
    FlashBwdLaunch f{};
    f.Q = Q;
    f.K = K;
    f.V = V;
    f.O = O;
    f.dO = dO;
    f.lse = lse;
    f.dQ = dQ;
    f.dK = dK;
    f.dV = dV;
    f.B = B;
    f.H = H;
    f.Hkv = Hkv;
    f.Sq = Sq;
    f.Sk = Sk;
    f.D = D;
    f.scale = scale;
    f.causal = causal != 0;
    return flash_bwd_run(f, workspace, workspace_bytes, stream);
}

int wmma_flash_attn_varlen_bwd(const void* dO, const void* Q, const void* K, const void* V,
                               const void* O, const float* lse, void* dQ, void* dK, void* dV,
                               const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                               void* workspace, size_t workspace_bytes, int B, int H, int Hkv,
                               int total_q, int total_k, int max_seqlen_q, int max_seqlen_k,
                               int D, float scale, int causal, void* stream) {
    if (int rc = flash_varlen_check(B, H, Hkv, total_q, total_k, max_seqlen_q, max_seqlen_k, D,
                                    scale, kFlashMaxDBwd))
        return rc;
    if (B == 0 || H == 0 || (total_q == 0 && total_k == 0)) return ok();
    if (!cu_seqlens_q || !cu_seqlens_k) return fail(WMMA_ERR_INVALID_ARG, "NULL pointer");
    if (!aligned4(cu_seqlens_q) || !aligned4(cu_seqlens_k))
        return fail(WMMA_ERR_MISALIGNED, "cu_seqlens must be 4-byte aligned");
    FlashBwdLaunch f{};
    f.Q = Q;
    f.K = K;
    f.V = V;
    f.O = O;
    f.dO = dO;
    f.lse = lse;
    f.dQ = dQ;
    f.dK = dK;
    f.dV = dV;
    f.B = B;
    f.H = H;
    f.Hkv = Hkv;
    f.Sq = max_seqlen_q;
    f.Sk = max_seqlen_k;
    f.D = D;
    f.scale = scale;
    f.causal = causal != 0;
    f.cu_q = cu_seqlens_q;
    f.cu_k = cu_seqlens_k;
    f.total_q = total_q;
    f.total_k = total_k;
    return flash_bwd_run(f, workspace, workspace_bytes, stream);
}

}  // extern "C"
