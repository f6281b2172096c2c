// Backend::matmul on the GPU (rust/src/backend/mod.rs:18-46): C[m,n] =
// A[m,k] B[k,n] in f32, row-major, bit-identical to the reference's x86 CPU
// backend (CpuBackend::matmul, rust/src/backend/cpu.rs:13-23, whose serial
// and rayon-split paths both run avx2_matmul, rust/src/kernels/simd.rs
// :226-249, on every row): for columns j < 8 floor(n / 8) each output starts
// at 0 and takes c = fma(a[i,l], b[l,j], c) for l = 0 .. k-1 in order; the
// n % 8 tail columns take c = c + a[i,l] * b[l,j] with the product rounded
// first (the scalar tail, simd.rs:240-247).  The order is sequential in k,
// so the parallelism is over outputs: one lane per column (a wave per 64
// columns), R rows of A per block as independent chains, A staged through
// LDS a window of k at a time, B's loads issued eight k-steps ahead.

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

}  // namespace

hipError_t launch_matmul_f32(const float *A, const float *B, float *C, int m, int k, int n,
                             hipStream_t st) {
    if (m <= 0 || n <= 0) return hipSuccess;
    if (m == 1) launch_rows<1>(A, B, C, m, k, n, st);
    else if (m == 2) launch_rows<2>(A, B, C, m, k, n, st);
    else if (m <= 4) launch_rows<4>(A, B, C, m, k, n, st);
    else launch_rows<8>(A, B, C, m, k, n, st);
    return hipGetLastError();
}

}  // namespace lcmoe
