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
// column, rows of A as independent chains.  The exact product
// (k_shard_matmul) decodes the weights ahead of the chains in other waves of
// the block; the k-sliced variant (k_shard_slice, short chains, many blocks)
// runs one wave per block.

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

constexpr int kShardCols = 64;   // columns per block: one lane per column
constexpr int kShardWaves = 8;   // waves per block: NC consumers, then producers
constexpr int kDqBufs = 3;       // decoded windows in LDS
constexpr int kShardMaxRows = 16;  // rows of A per block, at most (NC * R)

__device__ __forceinline__ void shard_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Block of 8 waves over 64 columns (two blocks of 32 along n) and NC * R rows
// of A.  The per-output chain is sequential in k, so the work splits by role:
//   * consumer waves 0 .. NC-1: lane j runs the R chains of column j, one
//     fused multiply-add per row and k-step, reading the decoded weights and
//     A from LDS (one LDS read per step, A broadcast);
//   * producer waves NC .. 7: stream the raw weight bytes and A with ordinary
//     loads L windows ahead (a ring of register sets, so a load has L windows
//     of the consumers' time to arrive), stage the raw rows in LDS and decode
//     them, q * scale rounded once as the reference, into the dq buffers.
// Window X (k-rows X W .. X W + W - 1) moves through the ticks of one loop
// with a block barrier per tick: at tick t the producers write window t's raw
// rows and A to LDS, decode window t - 1, and issue the loads of window t + L;
// the consumers run window t - 2.  Three dq / A buffers and two raw buffers
// keep every LDS write one barrier away from the reads of the same buffer.
// Results are exactly those of the one-wave kernel it replaces: each output
// is c = fma(a[i,l], dq[l,j], c) for l = 0 .. k-1 in order, from 0.
template <int QT, int NC, int R, int L, int kShardWin>
__global__ __launch_bounds__(64 * kShardWaves) void k_shard_matmul(
    const float *__restrict__ a, const uint8_t *__restrict__ b, float *__restrict__ c, int m,
    int kt, int n, int ks) {
    constexpr int BB = QT == LCMOE_TYPE_Q8_0 ? 34 : 18;  // bytes per block
    constexpr int UW = BB;                               // u16 per window row (two blocks)
    constexpr int NP = kShardWaves - NC;                 // producer waves
    constexpr int NPT = 64 * NP;                         // producer threads
    constexpr int NRAW = (kShardWin * UW + NPT - 1) / NPT;      // raw u16 loads per thread
    constexpr int NA = (NC * R * kShardWin + NPT - 1) / NPT;    // A loads per thread
    static_assert(L * (NRAW + NA) <= 63, "loads in flight past the vmcnt range");
    static_assert(NC * R <= kShardMaxRows, "rows per block");
    // the producers' raw and A buffers hold every element of their loads
    // (the ones past the window's bytes or the block's rows are padding), so
    // that staging them takes no per-lane branch
    // Raw window in LDS: the codes of each row's two blocks (CB bytes, so a
    // lane's four columns are one aligned read), then the rows' two scales,
    // then a slot the padding loads write to.
    constexpr int CB = QT == LCMOE_TYPE_Q8_0 ? 64 : 32;           // code bytes per row
    constexpr int RAWB = kShardWin * CB + kShardWin * 4 + 16;     // bytes per raw buffer
    constexpr int AROWS = (NA * NPT + kShardWin - 1) / kShardWin;  // rows the A loads cover
    static_assert(AROWS >= NC * R, "A staging rows");
    __shared__ __attribute__((aligned(16))) float s_dq[kDqBufs][kShardWin][kShardCols];
    __shared__ __attribute__((aligned(16))) float s_a[kDqBufs][AROWS][kShardWin];
    __shared__ __attribute__((aligned(16))) uint8_t s_raw[2][RAWB];

    // blockIdx.z: k slice [z ks, z ks + ks) into its own C plane (one slice:
    // the whole k straight into C)
    const int lda = kt, kz = blockIdx.z * ks, k = min(ks, kt - kz);
    a += kz;
    b += (int64_t)kz * (n >> 5) * BB;
    c += (int64_t)blockIdx.z * m * n;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, j = blockIdx.x * kShardCols + lane;
    const int i0 = blockIdx.y * (NC * R), mt = min(NC * R, m - i0);
    // k >= 1 (the host fills C with zeros for k = 0, and every k slice has
    // rows); the ticks run to a multiple of L so that every producer tick
    // issues its loads (below)
    const int NW = (k + kShardWin - 1) / kShardWin, NT = (NW + 2 + L - 1) / L * L;

    if (wave < NC) {
        // ---- consumer: R chains per lane -------------------------------------
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = 0.0f;
        for (int t = 0; t < NT; t++) {
            if (t >= 2 && t < NW + 2) {
                const int X = t - 2, bq = X % kDqBufs;
                const int wn = min(kShardWin, k - X * kShardWin);
                const float *dq = &s_dq[bq][0][lane];
                const float *ar = &s_a[bq][wave * R][0];
                if (R == 1 && wn == kShardWin) {
                    // one chain per lane: each step issues the reads of the
                    // step kAhead later (in-order LDS returns, so every wait
                    // leaves the younger reads in flight), filling the
                    // dependent multiply-add's latency
                    constexpr int kAhead = 16;
                    const float4 *a4 = reinterpret_cast<const float4 *>(ar);
                    float qv[kShardWin];
                    float4 av[kShardWin / 4];
#pragma unroll
                    for (int u = 0; u < kAhead; u++) {
                        qv[u] = dq[u * kShardCols];
                        if (u % 4 == 0) av[u / 4] = a4[u / 4];
                    }
#pragma unroll
                    for (int u = 0; u < kShardWin; u++) {
                        const int un = u + kAhead;
                        if (un < kShardWin) {
                            qv[un] = dq[un * kShardCols];
                            if (un % 4 == 0) av[un / 4] = a4[un / 4];
                        }
                        const float4 v = av[u / 4];
                        const float x = (u & 3) == 0 ? v.x : (u & 3) == 1 ? v.y
                                      : (u & 3) == 2 ? v.z : v.w;
                        acc[0] = __builtin_fmaf(x, qv[u], acc[0]);
                    }
                } else if (wn == kShardWin) {
                    // a full window in groups of 16 steps, each group's LDS
                    // reads issued before the previous group's multiply-adds
                    float qv[2][16];
                    float4 av[2][R][4];
                    auto fetch = [&](int g, float (&qd)[16], float4 (&ad)[R][4]) {
#pragma unroll
                        for (int u = 0; u < 16; u++) qd[u] = dq[(16 * g + u) * kShardCols];
#pragma unroll
                        for (int r = 0; r < R; r++)
#pragma unroll
                            for (int v = 0; v < 4; v++)
                                ad[r][v] = *reinterpret_cast<const float4 *>(
                                    ar + r * kShardWin + 16 * g + 4 * v);
                    };
                    fetch(0, qv[0], av[0]);
#pragma unroll
                    for (int g = 0; g < kShardWin / 16; g++) {
                        if (g + 1 < kShardWin / 16) fetch(g + 1, qv[(g + 1) & 1], av[(g + 1) & 1]);
#pragma unroll
                        for (int u = 0; u < 16; u++)
#pragma unroll
                            for (int r = 0; r < R; r++) {
                                const float4 v = av[g & 1][r][u >> 2];
                                const float x = (u & 3) == 0 ? v.x : (u & 3) == 1 ? v.y
                                              : (u & 3) == 2 ? v.z : v.w;
                                acc[r] = __builtin_fmaf(x, qv[g & 1][u], acc[r]);
                            }
                    }
                } else {
                    for (int w = 0; w < wn; w++) {
                        const float q = dq[w * kShardCols];
#pragma unroll
                        for (int r = 0; r < R; r++)
                            acc[r] = __builtin_fmaf(ar[r * kShardWin + w], q, acc[r]);
                    }
                }
            }
            shard_barrier();
        }
        if (j < n) {
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int row = wave * R + r;
                if (row < mt) c[(int64_t)(i0 + row) * n + j] = acc[r];
            }
        }
        return;
    }

    // ---- producers -----------------------------------------------------------
    const int q = (wave - NC) * 64 + lane;  // producer thread index
    const int nblk = min(2, (n >> 5) - 2 * (int)blockIdx.x);  // blocks of this group per row
    const int ug = nblk * BB / 2;                               // valid u16 per row
    const int64_t rs2 = (int64_t)(n >> 5) * BB / 2;             // u16 per k-row
    const uint16_t *pg = reinterpret_cast<const uint16_t *>(b + (int64_t)blockIdx.x * 2 * BB);
    // Per load i of this thread (window-independent): the window row w and
    // u16 u of its element, its offset from the window's first row, and its
    // byte offset in a raw LDS buffer (codes, scales, or the padding slot).
    int rw_row[NRAW];
    uint32_t src_off[NRAW], dst_off[NRAW];
#pragma unroll
    for (int i = 0; i < NRAW; i++) {
        const int e = q + NPT * i, w = min(e / UW, kShardWin - 1), u = e % UW;
        const int ub = BB / 2, g = u / ub, v = u % ub;  // block, u16 within the block
        rw_row[i] = w;
        src_off[i] = (uint32_t)(w * rs2 + min(u, ug - 1));
        dst_off[i] = e >= kShardWin * UW ? (uint32_t)(RAWB - 16)
                     : v == 0 ? (uint32_t)(kShardWin * CB + (2 * w + g) * 2)
                              : (uint32_t)(w * CB + g * (CB / 2) + 2 * (v - 1));
    }
    // A loads: row r and column w of element e; a pointer to its row
    const float *a_row[NA];
    int a_r[NA], a_w[NA];
#pragma unroll
    for (int i = 0; i < NA; i++) {
        const int e = q + NPT * i;
        a_r[i] = e / kShardWin;
        a_w[i] = e % kShardWin;
        a_row[i] = a + (int64_t)(i0 + min(a_r[i], mt - 1)) * lda;
    }
    uint32_t rr[L][NRAW];
    float ra[L][NA];
    // Window X's loads, every one unconditional: the window (past the last,
    // at the end of the ticks), the u16 past a ragged group of one block and
    // rows past k (the last window) are clamped to elements in bounds whose
    // values are never used (A: replaced by 0).  Every tick issuing the same
    // loads, branch-free, keeps each wait the compiler places a vmcnt(N) that
    // leaves the younger windows' loads in flight.
    auto issue = [&](int X, uint32_t (&rw)[NRAW], float (&av)[NA]) {
        const int l0 = min(X, NW - 1) * kShardWin;
        const uint16_t *base = pg + l0 * rs2;
        const int last = k - 1 - l0;  // window rows past it are past k
#pragma unroll
        for (int i = 0; i < NRAW; i++) {
            const int over = max(rw_row[i] - last, 0);
            rw[i] = base[src_off[i] - (uint32_t)(over * rs2)];
        }
#pragma unroll
        for (int i = 0; i < NA; i++) av[i] = a_row[i][l0 + min(a_w[i], last)];
    };
    auto stage = [&](int X, const uint32_t (&rw)[NRAW], const float (&av)[NA]) {
        uint8_t *raw = s_raw[X & 1];
#pragma unroll
        for (int i = 0; i < NRAW; i++)
            *reinterpret_cast<uint16_t *>(raw + dst_off[i]) = (uint16_t)rw[i];
        const int l0 = X * kShardWin;
#pragma unroll
        for (int i = 0; i < NA; i++)
            s_a[X % kDqBufs][a_r[i]][a_w[i]] = a_r[i] < mt && l0 + a_w[i] < k ? av[i] : 0.0f;
    };
    // Window X's values q * scale (one rounding, as the reference): one wave
    // op covers four rows, lane l taking row 4 o + l / 16 and the four columns
    // 4 (l % 16) .. +3 (one aligned LDS read of their codes), written to the
    // dq buffer as one 16-byte store.  All rows of the window, also those past
    // k in the last one (stale bytes, never read by the consumers).
    constexpr int OPS = kShardWin / 4, OPP = (OPS + NP - 1) / NP;  // ops, ops per producer
    auto decode = [&](int X) {
        const uint8_t *raw = s_raw[X & 1];
        const int c0 = 4 * (lane & 15), g = c0 >> 5;
        uint32_t cw[OPP], sw[OPP];
#pragma unroll
        for (int o = 0; o < OPP; o++) {
            const int w = 4 * min(wave - NC + NP * o, OPS - 1) + (lane >> 4);
            if constexpr (QT == LCMOE_TYPE_Q8_0)
                cw[o] = *reinterpret_cast<const uint32_t *>(raw + w * CB + c0);
            else
                cw[o] = *reinterpret_cast<const uint16_t *>(raw + w * CB + g * 16 + ((c0 & 31) >> 1));
            sw[o] = *reinterpret_cast<const uint16_t *>(raw + kShardWin * CB + (2 * w + g) * 2);
        }
#pragma unroll
        for (int o = 0; o < OPP; o++) {
            const int op = wave - NC + NP * o;
            const int w = 4 * op + (lane >> 4);
            const float d = dh2f(sw[o]);
            float4 v;
            if constexpr (QT == LCMOE_TYPE_Q8_0) {
                v.x = (float)(int8_t)(cw[o] & 0xffu) * d;
                v.y = (float)(int8_t)((cw[o] >> 8) & 0xffu) * d;
                v.z = (float)(int8_t)((cw[o] >> 16) & 0xffu) * d;
                v.w = (float)(int8_t)(cw[o] >> 24) * d;
            } else {  // element 2t: low nibble of byte t, 2t + 1: the high one
                v.x = (float)((int)(cw[o] & 15u) - 8) * d;
                v.y = (float)((int)((cw[o] >> 4) & 15u) - 8) * d;
                v.z = (float)((int)((cw[o] >> 8) & 15u) - 8) * d;
                v.w = (float)((int)((cw[o] >> 12) & 15u) - 8) * d;
            }
            if (op < OPS) *reinterpret_cast<float4 *>(&s_dq[X % kDqBufs][w][c0]) = v;
        }
    };
    // the prologue's windows in order (the scheduler may not interleave
    // them): each wait below then leaves exactly the younger windows in flight
#pragma unroll
    for (int s = 0; s < L; s++) {
        issue(s, rr[s], ra[s]);
        __builtin_amdgcn_sched_barrier(0);
    }
    for (int t0 = 0; t0 < NT; t0 += L) {
#pragma unroll
        for (int s = 0; s < L; s++) {
            const int t = t0 + s;
            if (t < NW) stage(t, rr[s], ra[s]);
            if (t >= 1 && t <= NW) decode(t - 1);
            issue(t + L, rr[s], ra[s]);
            shard_barrier();
        }
    }
}

constexpr int kSliceRows = 8;    // rows of A per block, at most

// k slices (lcmoe_shard_matmul_split*): one wave per block.  A slice's
// chain is short (k / S steps), so this kernel takes its parallelism from
// many small blocks.  Per window the wave fetches kSliceWin k-rows of its
// two (or, at a ragged end, one) blocks per row with 2-byte loads spread over
// the lanes, and the A window, into registers; they are written to LDS after
// the previous window has been consumed from the other buffer, so a window's
// loads are in flight while the one before it is computed.
// R rows of A per block (1, 2, 4 or 8): every chain runs unguarded (A rows
// past m are zeros in LDS) and only rows < m are stored.
template <int QT, int R, int kSliceWin, bool BATCH>
__global__ __launch_bounds__(kShardCols) void k_shard_slice(const float *__restrict__ a,
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
    constexpr int NB = kSliceWin * UG / kShardCols;      // u16 loads per lane per window
    constexpr int NA = R * kSliceWin / kShardCols;       // A loads per lane per window
    __shared__ uint16_t s_b[2][kSliceWin * UG];
    __shared__ float s_a[2][R * kSliceWin];
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
            const int e = lane + kShardCols * i, r = e / kSliceWin, w = e % kSliceWin;
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
    for (int l0 = 0; l0 < k; l0 += kSliceWin, buf ^= 1) {
        const bool more = l0 + kSliceWin < k;
        if (more) fetch(l0 + kSliceWin);
        if (col) {
            const uint8_t *sb = reinterpret_cast<const uint8_t *>(s_b[buf]) + g * BB;
            const int wn = min(kSliceWin, k - l0);
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
                    acc[r] = __builtin_fmaf(s_a[buf][r * kSliceWin + w], dq, acc[r]);
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
        hipLaunchKernelGGL((k_shard_slice<LCMOE_TYPE_Q8_0, R, W, true>), grid, dim3(kShardCols), 0, st, a,
                           b, c, m, k, n, ks);
    else
        hipLaunchKernelGGL((k_shard_slice<LCMOE_TYPE_Q4_0, R, W, (R > 1)>), grid, dim3(kShardCols), 0, st, a,
                           b, c, m, k, n, ks);
}

// (NC consumer waves, R rows each) by m; windows of 128 k-rows where the
// LDS allows (one or two rows of A), else 64; the register ring of raw
// loads (L windows) as deep as the vmcnt counter allows for that shape
template <int QT>
static void launch_cfg(const float *a, const uint8_t *b, float *c, int m, int k, int n, int S,
                       hipStream_t st) {
    const int ks = (k + S - 1) / S;
    auto go = [&](auto kern, int rows) {
        const dim3 grid((n + kShardCols - 1) / kShardCols, (m + rows - 1) / rows, S);
        hipLaunchKernelGGL(kern, grid, dim3(64 * kShardWaves), 0, st, a, b, c, m, k, n, ks);
    };
    if (m == 1) go(k_shard_matmul<QT, 1, 1, 4, 128>, 1);
    else if (m == 2) go(k_shard_matmul<QT, 2, 1, 4, 128>, 2);
    else if (m <= 4) go(k_shard_matmul<QT, 4, 1, 6, 64>, 4);
    else if (m <= 8) go(k_shard_matmul<QT, 4, 2, 5, 64>, 8);
    else go(k_shard_matmul<QT, 4, 4, 4, 64>, 16);
}

__global__ __launch_bounds__(256) void k_shard_zero(float *__restrict__ c, int64_t count) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < count) c[i] = 0.0f;
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
    if (k == 0) {  // empty sums: C = 0
        const int64_t count = (int64_t)m * n;
        hipLaunchKernelGGL(k_shard_zero, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, st,
                           c, count);
        return hipGetLastError();
    }
    if (S == 1) {
        if (qt == LCMOE_TYPE_Q8_0)
            launch_cfg<LCMOE_TYPE_Q8_0>(a, b, c, m, k, n, 1, st);
        else
            launch_cfg<LCMOE_TYPE_Q4_0>(a, b, c, m, k, n, 1, st);
        return hipGetLastError();
    }
    // k slices into ws; a window of kSliceWin k-rows, longer for one row of
    // A, whose chains are too short per row to cover a window's loads
    // otherwise
    if (m == 1) launch_rows<1, 128>(qt, a, b, ws, m, k, n, S, st);
    else if (m == 2) launch_rows<2, 64>(qt, a, b, ws, m, k, n, S, st);
    else if (m <= 4) launch_rows<4, 64>(qt, a, b, ws, m, k, n, S, st);
    else launch_rows<kSliceRows, 64>(qt, a, b, ws, m, k, n, S, st);
    const int64_t plane = (int64_t)m * n;
    hipLaunchKernelGGL(k_shard_reduce, dim3((unsigned)((plane + 255) / 256)), dim3(256), 0, st, ws,
                       S, plane, c);
    return hipGetLastError();
}

}  // namespace lcmoe
