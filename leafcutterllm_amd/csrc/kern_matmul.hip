// Backend::matmul on the GPU (rust/src/backend/mod.rs:18-46): C[m,n] =
// A[m,k] B[k,n] in f32, row-major, bit-identical to the reference's x86 CPU
// backend (CpuBackend::matmul, rust/src/backend/cpu.rs:13-23, whose serial
// and rayon-split paths both run avx2_matmul, rust/src/kernels/simd.rs
// :226-249, on every row): for columns j < 8 floor(n / 8) each output starts
// at 0 and takes c = fma(a[i,l], b[l,j], c) for l = 0 .. k-1 in order; the
// n % 8 tail columns take c = c + a[i,l] * b[l,j] with the product rounded
// first (the scalar tail, simd.rs:240-247).  The order is sequential in k,
// so the parallelism is over outputs: one lane per output column, R rows of
// A per lane as independent chains.
//
// Two kernels:
//   * k_matmul_stream (n % 4 == 0, B 16-byte aligned): blocks of consumer
//     waves that run the chains out of LDS and producer waves that stream B
//     and A into LDS several k-windows ahead.  Small m takes blocks of 16
//     columns (four row groups of 16 lanes per wave) so that a 4096-column
//     product spreads over 256 blocks and each block needs only a modest
//     number of bytes in flight to keep HBM busy;
//   * k_matmul_f32 (any shape): one wave per 64 columns, A staged through
//     LDS a window at a time, B loaded eight k-steps ahead.

#include <cstdint>
#include <type_traits>

#include "device_common.h"
#include "kernels.h"

namespace lcmoe {
namespace {

constexpr int kMmCols = 64;   // columns per block (one wave)
constexpr int kMmWin = 256;   // k-steps of A per LDS window

template <int R>
__global__ __launch_bounds__(kMmCols) void k_matmul_f32(const float *__restrict__ A,
                                                        const float *__restrict__ B,
                                                        float *__restrict__ C, int m, int k, int n,
                                                        int n8) {
    __shared__ float s_a[R * kMmWin];
    const int lane = threadIdx.x, j = blockIdx.x * kMmCols + lane;
    const int i0 = blockIdx.y * R, mt = min(R, m - i0);
    const bool col = j < n, fused = j < n8;
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
    const float *bj = B + (col ? j : 0);
    for (int l0 = 0; l0 < k; l0 += kMmWin) {
        const int wn = min(kMmWin, k - l0);
        // the window of A: rows past m are zeros (their chains are not stored)
        for (int e = lane; e < R * kMmWin; e += kMmCols) {
            const int r = e / kMmWin, w = e % kMmWin;
            s_a[e] = r < mt && w < wn ? A[(int64_t)(i0 + r) * k + l0 + w] : 0.0f;
        }
        __syncthreads();
        if (col) {
            int w = 0;
            for (; w + 8 <= wn; w += 8) {
                float b[8];
#pragma unroll
                for (int u = 0; u < 8; u++) b[u] = bj[(int64_t)(l0 + w + u) * n];
#pragma unroll
                for (int u = 0; u < 8; u++)
#pragma unroll
                    for (int r = 0; r < R; r++) {
                        const float av = s_a[r * kMmWin + w + u];
                        if (fused) {
                            acc[r] = __builtin_fmaf(av, b[u], acc[r]);
                        } else {
                            const float p = av * b[u];
                            acc[r] = acc[r] + p;
                        }
                    }
            }
            for (; w < wn; w++) {
                const float bv = bj[(int64_t)(l0 + w) * n];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const float av = s_a[r * kMmWin + w];
                    if (fused) {
                        acc[r] = __builtin_fmaf(av, bv, acc[r]);
                    } else {
                        const float p = av * bv;
                        acc[r] = acc[r] + p;
                    }
                }
            }
        }
        __syncthreads();
    }
    if (!col) return;
#pragma unroll
    for (int r = 0; r < R; r++)
        if (r < mt) C[(int64_t)(i0 + r) * n + j] = acc[r];
}

template <int R>
void launch_rows(const float *A, const float *B, float *C, int m, int k, int n, hipStream_t st) {
    const dim3 grid((n + kMmCols - 1) / kMmCols, (m + R - 1) / R);
    hipLaunchKernelGGL(k_matmul_f32<R>, grid, dim3(kMmCols), 0, st, A, B, C, m, k, n, n & ~7);
}

typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void mm_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// One k-window of a consumer lane's R chains: wn steps, b from the lane's
// column of the B window (BT: the column's own LDS row, contiguous in k;
// else stride CB), a from R rows of the A window (stride WP).  FUSED: c = fma(a, b, c) (the first 8 floor(n / 8) columns); else
// c = c + a * b with the product rounded first (the tail columns).  A full
// window reads LDS in groups of GS steps: group g + 1's reads are issued
// (scheduling barriers keep them there) before group g's multiply-adds, so
// each read has a group of dependent multiply-adds' time to return, and at
// most 12 reads are in flight (the LDS counter's range is 15).
template <int CB, int R, int W, int WP, bool FUSED, bool BT>
__device__ __forceinline__ void mm_window(const float *sb, const float *sa, int wn,
                                          float (&acc)[R]) {
    auto upd = [&](float a, float b, float &c) {
        if constexpr (FUSED) {
            c = __builtin_fmaf(a, b, c);
        } else {
            const float p = a * b;
            c = c + p;
        }
    };
    if (wn == W) {
        // reads per group: GS / 4 float4 (BT) or GS / 2 pairs (one ds_read2
        // each) of B values, and R * GS / 4 float4 of A
        constexpr int GS = R >= 4 ? 8 : R == 2 ? 8 : 16;
        static_assert((BT ? GS / 4 : GS / 2) + R * GS / 4 <= 12, "reads in flight per group");
        float bq[2][GS];
        v4f aq[2][R][GS / 4];
        auto fetch = [&](int gi, float (&bd)[GS], v4f (&ad)[R][GS / 4]) {
            if constexpr (BT) {
#pragma unroll
                for (int v = 0; v < GS / 4; v++) {
                    const v4f x = *reinterpret_cast<const v4f *>(sb + GS * gi + 4 * v);
                    bd[4 * v] = x[0];
                    bd[4 * v + 1] = x[1];
                    bd[4 * v + 2] = x[2];
                    bd[4 * v + 3] = x[3];
                }
            } else {
#pragma unroll
                for (int u = 0; u < GS; u++) bd[u] = sb[(GS * gi + u) * CB];
            }
#pragma unroll
            for (int r = 0; r < R; r++)
#pragma unroll
                for (int v = 0; v < GS / 4; v++)
                    ad[r][v] = *reinterpret_cast<const v4f *>(sa + r * WP + GS * gi + 4 * v);
        };
        fetch(0, bq[0], aq[0]);
#pragma unroll
        for (int gi = 0; gi < W / GS; gi++) {
            if (gi + 1 < W / GS) fetch(gi + 1, bq[(gi + 1) & 1], aq[(gi + 1) & 1]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < GS; u++)
#pragma unroll
                for (int r = 0; r < R; r++) upd(aq[gi & 1][r][u >> 2][u & 3], bq[gi & 1][u], acc[r]);
            __builtin_amdgcn_sched_barrier(0);
        }
    } else {
        for (int w = 0; w < wn; w++) {
            const float b = sb[BT ? w : w * CB];
#pragma unroll
            for (int r = 0; r < R; r++) upd(sa[r * WP + w], b, acc[r]);
        }
    }
}

// Streaming product for n % 4 == 0 and B 16-byte aligned.  A block covers
// CB columns and RB = NC (64 / CB) R rows of A; its waves split by role:
//   * consumer waves 0 .. NC-1: lane l takes column j0 + l % CB and the R
//     rows of its row group l / CB, one chain per row, reading B and A from
//     the LDS window;
//   * producer waves NC .. NC+NP-1: load window X (k-rows X W .. X W + W - 1)
//     of B (float4 per load) and of A (float4 when AV: k % 4 == 0 and A
//     16-byte aligned) into registers L windows ahead, and store them to LDS.
// Window X moves through the ticks of one loop with one block barrier per
// tick: at tick t the producers store window t into LDS buffer t & 1 and
// issue the loads of window t + L; the consumers run window t - 1 from the
// other buffer.  Loads past k, past n or past m are clamped to elements in
// bounds: their values land in LDS slots no stored chain reads (the chains
// stop at k; columns past n and rows past m are not stored).  Every tick
// issues the same loads, branch-free, so each wait the compiler places
// leaves the younger windows' loads in flight.
// Columns: blocks of CB over the first n8 = 8 floor(n / 8) (the last one
// ragged), then, when n8 < n, one block of the four tail columns, so that
// every block runs one update rule.  Block order: with the block count a
// multiple of 8, block b (dispatched to XCD b % 8) takes tile
// (b % 8) (count / 8) + b / 8, so each XCD's L2 holds a contiguous range of
// columns (adjacent 16-column blocks share B's cache lines); the row blocks
// of one column block are adjacent tiles.
template <int CB, int NC, int R, int NP, int W, int L, bool AV>
__global__ __launch_bounds__(64 * (NC + NP)) void k_matmul_stream(
    const float *__restrict__ A, const float *__restrict__ B, float *__restrict__ C, int m, int k,
    int n, int n8, int nrb, int xcd_per) {
    constexpr int G = 64 / CB;                   // row groups per consumer wave
    constexpr int RB = NC * G * R;               // rows of A per block
    constexpr int WP = W + 4;                    // A row stride in LDS (spreads the groups' banks)
    // 16-column blocks hold B transposed in LDS (a column's W values
    // contiguous, rows W + 4 apart: a consumer reads four k-steps with one
    // float4, and a producer's four column stores from one float4 fall on
    // distinct banks pairwise)
    constexpr bool BT = CB == 16;
    constexpr int SB = BT ? CB * WP : W * CB;    // floats per B buffer
    constexpr int NPT = 64 * NP;                 // producer threads
    constexpr int BV = W * CB / 4;               // float4 of B per window
    constexpr int NB = BV / NPT;                 // ... per producer thread
    constexpr int AE = AV ? RB * W / 4 : RB * W; // A loads per window
    constexpr int NA = (AE + NPT - 1) / NPT;     // ... per producer thread
    static_assert(BV % NPT == 0, "the B window splits evenly over the producers");
    static_assert(L * (NB + NA) <= 60, "loads in flight within the vmcnt range");
    using AT = typename std::conditional<AV, v4f, float>::type;
    __shared__ __attribute__((aligned(16))) float s_b[2][SB];
    __shared__ __attribute__((aligned(16))) float s_a[2][RB * WP];

    int tile = blockIdx.x;
    if (xcd_per) tile = (blockIdx.x & 7) * xcd_per + (blockIdx.x >> 3);
    const int i0 = (tile % nrb) * RB, cb = tile / nrb;
    const int nfb = (n8 + CB - 1) / CB;                       // fused column blocks
    const bool tail = cb == nfb;                              // the tail block
    const int j0 = tail ? n8 : cb * CB, jend = tail ? n : min(j0 + CB, n8);
    // k >= 1; NW windows, ticks to a multiple of L past the last window's
    // consumption (every producer tick issues its loads)
    const int NW = (k + W - 1) / W, NT = (NW + L) / L * L;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;

    if (wave < NC) {
        const int c = lane % CB, rb = (wave * G + lane / CB) * R, j = j0 + c;
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] = 0.0f;
        for (int t = 0; t < NT; t++) {
            if (t >= 1 && t <= NW) {
                const int X = t - 1, wn = min(W, k - X * W);
                const float *sb = s_b[X & 1] + (BT ? c * WP : c), *sa = s_a[X & 1] + rb * WP;
                if (tail) mm_window<CB, R, W, WP, false, BT>(sb, sa, wn, acc);
                else mm_window<CB, R, W, WP, true, BT>(sb, sa, wn, acc);
            }
            mm_barrier();
        }
        if (j < jend) {
#pragma unroll
            for (int r = 0; r < R; r++)
                if (i0 + rb + r < m) C[(int64_t)(i0 + rb + r) * n + j] = acc[r];
        }
        return;
    }

    // ---- producers -----------------------------------------------------------
    const int q = (wave - NC) * 64 + lane;
    // B float4 e = q + NPT i of a window: k-row e / (CB / 4), columns
    // j0 + 4 (e % (CB / 4)) .. +3, clamped into the block's columns (jend is
    // a multiple of 4); in LDS at float 4 e (row-major [W][CB]) or, BT, at
    // [column][k-row]
    int b_w[NB], b_col[NB];
#pragma unroll
    for (int i = 0; i < NB; i++) {
        const int e = q + NPT * i;
        b_w[i] = e / (CB / 4);
        b_col[i] = min(j0 + 4 * (e % (CB / 4)), jend - 4);
    }
    // A load e = q + NPT i: row r of the block, k offset w in the window
    const float *a_row[NA];
    int a_r[NA], a_w[NA];
#pragma unroll
    for (int i = 0; i < NA; i++) {
        const int e = min(q + NPT * i, AE - 1);
        a_r[i] = AV ? e / (W / 4) : e / W;
        a_w[i] = AV ? 4 * (e % (W / 4)) : e % W;
        a_row[i] = A + (int64_t)min(i0 + a_r[i], m - 1) * k;
    }
    v4f rbv[L][NB];
    AT rav[L][NA];
    auto issue = [&](int X, v4f (&bv)[NB], AT (&av)[NA]) {
        const int l0 = min(X, NW - 1) * W;
#pragma unroll
        for (int i = 0; i < NB; i++)
            bv[i] = *reinterpret_cast<const v4f *>(B + (int64_t)min(l0 + b_w[i], k - 1) * n +
                                                      b_col[i]);
#pragma unroll
        for (int i = 0; i < NA; i++) {
            if constexpr (AV)  // k % 4 == 0: a float4 lies wholly before k or past it
                av[i] = *reinterpret_cast<const v4f *>(a_row[i] + min(l0 + a_w[i], k - 4));
            else
                av[i] = a_row[i][min(l0 + a_w[i], k - 1)];
        }
    };
    auto stage = [&](int X, const v4f (&bv)[NB], const AT (&av)[NA]) {
        float *sb = s_b[X & 1], *sa = s_a[X & 1];
#pragma unroll
        for (int i = 0; i < NB; i++) {
            if constexpr (BT) {
                const int e = q + NPT * i, c0 = 4 * (e % (CB / 4));
#pragma unroll
                for (int x = 0; x < 4; x++) sb[(c0 + x) * WP + b_w[i]] = bv[i][x];
            } else {
                *reinterpret_cast<v4f *>(sb + 4 * (q + NPT * i)) = bv[i];
            }
        }
#pragma unroll
        for (int i = 0; i < NA; i++)
            if (AE % NPT == 0 || q + NPT * i < AE)
                *reinterpret_cast<AT *>(sa + a_r[i] * WP + a_w[i]) = av[i];
    };
    // the prologue's windows in order (the scheduler may not interleave
    // them): each wait below then leaves exactly the younger windows in flight
#pragma unroll
    for (int s = 0; s < L; s++) {
        issue(s, rbv[s], rav[s]);
        __builtin_amdgcn_sched_barrier(0);
    }
    for (int t0 = 0; t0 < NT; t0 += L) {
#pragma unroll
        for (int s = 0; s < L; s++) {
            const int t = t0 + s;
            if (t < NW) stage(t, rbv[s], rav[s]);
            issue(t + L, rbv[s], rav[s]);
            mm_barrier();
        }
    }
}

// Launches k_matmul_stream over the whole product; false (nothing launched)
// when its tile count does not fit one grid dimension.
template <int CB, int NC, int R, int NP, int W, int L>
bool launch_stream(const float *A, const float *B, float *C, int m, int k, int n,
                   hipStream_t st) {
    constexpr int RB = NC * (64 / CB) * R;
    const int nrb = (m + RB - 1) / RB;
    const int n8 = n & ~7;
    const int64_t nb = (int64_t)nrb * ((n8 + CB - 1) / CB + (n8 < n ? 1 : 0));
    if (nb >= (1ll << 31)) return false;
    const int xcd_per = nb % 8 == 0 ? (int)(nb / 8) : 0;
    const dim3 grid((unsigned)nb), block(64 * (NC + NP));
    if (k % 4 == 0 && ((uintptr_t)A & 15) == 0)
        hipLaunchKernelGGL((k_matmul_stream<CB, NC, R, NP, W, L, true>), grid, block, 0, st, A, B,
                           C, m, k, n, n8, nrb, xcd_per);
    else
        hipLaunchKernelGGL((k_matmul_stream<CB, NC, R, NP, W, L, false>), grid, block, 0, st, A, B,
                           C, m, k, n, n8, nrb, xcd_per);
    return true;
}

}  // namespace

hipError_t launch_matmul_f32(const float *A, const float *B, float *C, int m, int k, int n,
                             hipStream_t st) {
    if (m <= 0 || n <= 0) return hipSuccess;
    if (k > 0 && n % 4 == 0 && ((uintptr_t)B & 15) == 0) {
        // m <= 16: 16-column blocks of one chain per lane, one chain wave per
        // four rows, four producer waves; wider m: 64-column blocks of four
        // chain waves (four rows per lane) and two producers
        const bool done = m <= 4    ? launch_stream<16, 1, 1, 4, 128, 4>(A, B, C, m, k, n, st)
                          : m <= 8  ? launch_stream<16, 2, 1, 4, 128, 4>(A, B, C, m, k, n, st)
                          : m <= 16 ? launch_stream<16, 4, 1, 4, 128, 4>(A, B, C, m, k, n, st)
                                    : launch_stream<64, 4, 4, 2, 64, 2>(A, B, C, m, k, n, st);
        if (done) return hipGetLastError();
    }
    if (m == 1) launch_rows<1>(A, B, C, m, k, n, st);
    else if (m == 2) launch_rows<2>(A, B, C, m, k, n, st);
    else if (m <= 4) launch_rows<4>(A, B, C, m, k, n, st);
    else launch_rows<8>(A, B, C, m, k, n, st);
    return hipGetLastError();
}

}  // namespace lcmoe
