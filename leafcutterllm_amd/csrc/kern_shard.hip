// The shard engine's quantised GEMM (rust/src/kernels/int8_gemm.rs),
// C[m,n] = A[m,k] B[k,n] with B stored as blocks of 32 along n, row-major
// over k: Q8_0 blocks of 34 bytes (f16 scale, 32 int8) or the shard Q4_0
// blocks of 18 bytes (f16 scale, 16 bytes; element 2t is the low nibble of
// byte t, 2t+1 the high one, value nibble - 8: q4_0.rs:36-46).
//
// Results are bit-identical to the x86 path the reference always takes for
// these shapes (q8_0_matmul_avx2_inner int8_gemm.rs:47-98, the Q4_0 twin
// :240-290): each output starts at 0 and takes, for l = 0 .. k-1 in order,
// c = fma(a[i,l], q * scale, c), the dequantised weight rounded once.  That
// order is sequential in k, so the parallelism is over outputs: one lane per
// column, kShardRows rows of A per block held as independent chains, the
// weights and A staged through LDS a window of kShardWin k-rows ahead.

#include <mutex>

#include "device_common.h"
#include "kernels.h"

namespace lcmoe {

// Scratch of lcmoe_shard_matmul_split_noalloc_dev: the k-slice planes
// [S, m, n].  Every GPU the library runs on holds its own copy until the
// process ends.  Host code never passes this name to a kernel (on the host it
// is a stand-in, not a device address); it uses the per-device address that
// shard_scratch() looks up.
static __device__ __align__(256) float scratch[kShardScratchFloats];

hipError_t shard_scratch(float **out) {
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static float *addr[kMaxDevices];
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        float *p = nullptr;
        e = hipGetSymbolAddress((void **)&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        addr[dev] = p;
    }
    *out = addr[dev];
    return hipSuccess;
}

namespace {

constexpr int kShardCols = 64;   // columns per block: one wave, one lane per column
constexpr int kShardRows = 8;    // rows of A per block, at most

// One wave per block.  Per window the wave fetches kShardWin k-rows of its
// two (or, at a ragged end, one) blocks per row with 2-byte loads spread over
// the lanes, and the A window, into registers; they are written to LDS after
// the previous window has been consumed from the other buffer, so a window's
// loads are in flight while the one before it is computed.
// R rows of A per block (1, 2, 4 or 8): every chain runs unguarded (A rows
// past m are zeros in LDS) and only rows < m are stored.
template <int QT, int R, int kShardWin, bool BATCH>
__global__ __launch_bounds__(kShardCols) void k_shard_matmul(const float *__restrict__ a,
                                                             const uint8_t *__restrict__ b,
                                                             float *__restrict__ c, int m, int kt,
                                                             int n, int ks) {
    // blockIdx.z: k slice [z ks, z ks + ks) into its own C plane (one slice:
    // the whole k straight into C)
    const int lda = kt, kz = blockIdx.z * ks, k = min(ks, kt - kz);
    a += kz;
    b += (int64_t)kz * (n >> 5) * (QT == LCMOE_TYPE_Q8_0 ? 34 : 18);
    c += (int64_t)blockIdx.z * m * n;
    constexpr int BB = QT == LCMOE_TYPE_Q8_0 ? 34 : 18;  // bytes per block
    constexpr int UG = BB;                               // u16 per k-row of two blocks
    constexpr int NB = kShardWin * UG / kShardCols;      // u16 loads per lane per window
    constexpr int NA = R * kShardWin / kShardCols;       // A loads per lane per window
    __shared__ uint16_t s_b[2][kShardWin * UG];
    __shared__ float s_a[2][R * kShardWin];
    const int lane = threadIdx.x, j = blockIdx.x * kShardCols + lane;
    const int i0 = blockIdx.y * R, mt = min(R, m - i0);
    const int nblk = min(2, (n >> 5) - 2 * (int)blockIdx.x);  // blocks of this group per row
    const int ug = nblk * BB / 2;                               // valid u16 per row
    const int64_t rs = (int64_t)(n >> 5) * BB;                  // bytes per k-row
    const uint16_t *pg = reinterpret_cast<const uint16_t *>(b + (int64_t)blockIdx.x * 2 * BB);
    const int g = lane >> 5, t = lane & 31;
    const bool col = j < n;
    uint16_t rb[NB];
    float ra[NA];
    auto fetch = [&](int l0) {
#pragma unroll
        for (int i = 0; i < NB; i++) {
            const int e = lane + kShardCols * i, w = e / UG, u = e % UG;
            if (l0 + w < k && u < ug) rb[i] = pg[((int64_t)(l0 + w) * rs >> 1) + u];
        }
#pragma unroll
        for (int i = 0; i < NA; i++) {
            const int e = lane + kShardCols * i, r = e / kShardWin, w = e % kShardWin;
            ra[i] = r < mt && l0 + w < k ? a[(int64_t)(i0 + r) * lda + l0 + w] : 0.0f;
        }
    };
    auto stage = [&](int buf) {
#pragma unroll
        for (int i = 0; i < NB; i++) s_b[buf][lane + kShardCols * i] = rb[i];
#pragma unroll
        for (int i = 0; i < NA; i++) s_a[buf][lane + kShardCols * i] = ra[i];
    };
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    fetch(0);
    stage(0);
    __syncthreads();
    int buf = 0;
    for (int l0 = 0; l0 < k; l0 += kShardWin, buf ^= 1) {
        const bool more = l0 + kShardWin < k;
        if (more) fetch(l0 + kShardWin);
        if (col) {
            const uint8_t *sb = reinterpret_cast<const uint8_t *>(s_b[buf]) + g * BB;
            const int wn = min(kShardWin, k - l0);
            // one row's scale and code from LDS
            auto read = [&](int w, uint32_t &sv, int32_t &qv) {
                const uint8_t *blk = sb + w * 2 * UG;
                sv = *reinterpret_cast<const uint16_t *>(blk);
                if constexpr (QT == LCMOE_TYPE_Q8_0) qv = (int8_t)blk[2 + t];
                else qv = blk[2 + (t >> 1)];
            };
            auto step = [&](int w, uint32_t sv, int32_t qv) {
                float q;
                if constexpr (QT == LCMOE_TYPE_Q8_0) q = (float)qv;
                else q = (float)((t & 1) ? (qv >> 4) : (qv & 15)) - 8.0f;
                const float dq = q * dh2f(sv);
#pragma unroll
                for (int r = 0; r < R; r++)
                    acc[r] = __builtin_fmaf(s_a[buf][r * kShardWin + w], dq, acc[r]);
            };
            int w = 0;
            if constexpr (!BATCH) {  // measured faster for one row of Q4_0
#pragma unroll 8
                for (; w < wn; w++) {
                    uint32_t sv;
                    int32_t qv;
                    read(w, sv, qv);
                    step(w, sv, qv);
                }
            }
            for (; w + 8 <= wn; w += 8) {  // eight rows' reads, then their steps in order
                uint32_t sv[8];
                int32_t qv[8];
#pragma unroll
                for (int u = 0; u < 8; u++) read(w + u, sv[u], qv[u]);
#pragma unroll
                for (int u = 0; u < 8; u++) step(w + u, sv[u], qv[u]);
            }
            for (; w < wn; w++) {
                uint32_t sv;
                int32_t qv;
                read(w, sv, qv);
                step(w, sv, qv);
            }
        }
        if (more) stage(buf ^ 1);  // the other buffer was last read before the barrier
        __syncthreads();
    }
    if (!col) return;
#pragma unroll
    for (int r = 0; r < R; r++)
        if (r < mt) c[(int64_t)(i0 + r) * n + j] = acc[r];
}

}  // namespace

template <int R, int W>
static void launch_rows(int qt, const float *a, const uint8_t *b, float *c, int m, int k, int n,
                        int S, hipStream_t st) {
    const int ks = (k + S - 1) / S;
    const dim3 grid((n + kShardCols - 1) / kShardCols, (m + R - 1) / R, S);
    if (qt == LCMOE_TYPE_Q8_0)
        hipLaunchKernelGGL((k_shard_matmul<LCMOE_TYPE_Q8_0, R, W, true>), grid, dim3(kShardCols), 0, st, a,
                           b, c, m, k, n, ks);
    else
        hipLaunchKernelGGL((k_shard_matmul<LCMOE_TYPE_Q4_0, R, W, (R > 1)>), grid, dim3(kShardCols), 0, st, a,
                           b, c, m, k, n, ks);
}

// C = the slices' planes added in slice order, from the first
__global__ __launch_bounds__(256) void k_shard_reduce(const float *__restrict__ ws, int S,
                                                      int64_t plane, float *__restrict__ c) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= plane) return;
    float s = ws[i];
    for (int z = 1; z < S; z++) s = s + ws[z * plane + i];
    c[i] = s;
}

hipError_t launch_shard_matmul(int qt, const float *a, const uint8_t *b, float *c, int m, int k,
                               int n, hipStream_t st, int S, float *ws) {
    float *dst = S > 1 ? ws : c;
    // a window of kShardWin k-rows: longer for one row of A, whose chains
    // are too short per row to cover a window's loads otherwise
    if (m == 1) launch_rows<1, 128>(qt, a, b, dst, m, k, n, S, st);
    else if (m == 2) launch_rows<2, 64>(qt, a, b, dst, m, k, n, S, st);
    else if (m <= 4) launch_rows<4, 64>(qt, a, b, dst, m, k, n, S, st);
    else launch_rows<kShardRows, 64>(qt, a, b, dst, m, k, n, S, st);
    if (S > 1) {
        const int64_t plane = (int64_t)m * n;
        hipLaunchKernelGGL(k_shard_reduce, dim3((unsigned)((plane + 255) / 256)), dim3(256), 0, st,
                           ws, S, plane, c);
    }
    return hipGetLastError();
}

}  // namespace lcmoe
