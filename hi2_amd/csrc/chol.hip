// Damped Cholesky chain of inverse_factor (hi2/hessian.py:71-86) on gfx950.
//
// The reference evaluates U = chol_upper(sym(cholesky_inverse(chol(H)))) with
// H = Hs + lam I: three O(K^3) passes (4K^3/3 flops).  The same matrix is
//   U = (J L J)^-1 = J L^-1 J,   L = chol(J H J),   J = the reversal permutation,
// because J L J is upper triangular with H = (J L J)(J L J)^T, so (J L J)^-1 is the
// upper triangular factor of H^-1 with positive diagonal, which is unique.  That is
// one Cholesky and one triangular inverse: 2K^3/3 flops.
//
// Blocked, right-looking, NB = 128:
//   potrf: per block column, a one-workgroup LDS factorisation (+ inverse) of the
//          diagonal block, the panel solve as a GEMM with that inverse, and the
//          trailing SYRK update on fp32 MFMA;
//   trtri: recursive, inv([A 0; B C]) = [A^-1 0; -C^-1 B A^-1  C^-1], leaves from the
//          diagonal inverses, the two products per node as triangular GEMMs.
#include <vector>

#include "common.h"

namespace hi2x {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int NB = 128;
constexpr int GT = 128, GK = 16;

// ---- generic fp32 MFMA GEMM ----------------------------------------------------------
// C[M, N] = alpha * A[M, Kd] * op(B) + beta * C, op(B) = B [Kd, N] (TB = false) or
// B^T with B [N, Kd] (TB = true).  Flags skip structural zeros at tile granularity:
//   ALOW: A lower triangular (A[i][k] = 0 for k > i)  -> k < row tile end
//   BLOW: op(B) lower triangular (op(B)[k][j] = 0 for k < j) -> k >= col tile start
//   CLOW: only the lower triangle of C (incl. diagonal) is computed and written.
struct GemmArgs {
  const float* A;
  const float* B;
  float* C;
  int64_t M, N, Kd, lda, ldb, ldc;
  float alpha, beta;
};

template <bool TB, bool ALOW, bool BLOW, bool CLOW>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs g) {
  __shared__ float As[GK][GT + 4];
  __shared__ float Bs[GK][GT + 4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = wave >> 1, wcn = wave & 1;
  const int64_t r0 = (int64_t)blockIdx.y * GT, c0 = (int64_t)blockIdx.x * GT;
  if (CLOW && c0 > r0 + GT - 1) return;
  int64_t kbeg = 0, kend = g.Kd;
  if (ALOW) kend = (r0 + GT < kend) ? r0 + GT : kend;
  if (BLOW) kbeg = c0 - (c0 % GK);
  f32x16 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[a][b][j] = 0.0f;
  for (int64_t k0 = kbeg; k0 < kend; k0 += GK) {
    __syncthreads();
    {  // A chunk: As[k][m] = A[r0+m, k0+k]
      const int m = tid >> 1, h = tid & 1;
      const int64_t rr = r0 + m;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int64_t kk = k0 + h * 8 + j;
        // ALOW: the strict upper triangle of A is structurally zero (not read)
        const bool ok = rr < g.M && kk < kend && (!ALOW || kk <= rr);
        As[h * 8 + j][m] = ok ? g.A[rr * g.lda + kk] : 0.0f;
      }
    }
    if (TB) {  // Bs[k][n] = B[c0+n, k0+k]
      const int n = tid >> 1, h = tid & 1;
      const int64_t cc = c0 + n;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int64_t kk = k0 + h * 8 + j;
        const bool ok = cc < g.N && kk < kend && (!BLOW || kk >= cc);
        Bs[h * 8 + j][n] = ok ? g.B[cc * g.ldb + kk] : 0.0f;
      }
    } else {  // Bs[k][n] = B[k0+k, c0+n]
      const int k = tid >> 4, nb = (tid & 15) * 8;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int64_t cc = c0 + nb + j, kk = k0 + k;
        // BLOW: op(B)[k][j] = 0 for k < j (not read)
        const bool ok = cc < g.N && kk < kend && (!BLOW || kk >= cc);
        Bs[k][nb + j] = ok ? g.B[kk * g.ldb + cc] : 0.0f;
      }
    }
    __syncthreads();
#pragma unroll
    for (int k2 = 0; k2 < GK; k2 += 2) {
      const int kr = k2 + (lane >> 5);
      float av[2], bv[2];
#pragma unroll
      for (int a = 0; a < 2; ++a) av[a] = As[kr][wr * 64 + a * 32 + (lane & 31)];
#pragma unroll
      for (int b = 0; b < 2; ++b) bv[b] = Bs[kr][wcn * 64 + b * 32 + (lane & 31)];
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[a], bv[b], acc[a][b], 0, 0, 0);
    }
  }
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int64_t row = r0 + wr * 64 + a * 32 + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
        const int64_t col = c0 + wcn * 64 + b * 32 + (lane & 31);
        if (row >= g.M || col >= g.N) continue;
        if (CLOW && col > row) continue;
        float* cp = g.C + row * g.ldc + col;
        const float v = g.alpha * acc[a][b][j];
        *cp = (g.beta != 0.0f) ? g.beta * *cp + v : v;
      }
}

template <bool TB, bool ALOW, bool BLOW, bool CLOW>
int gemm(const GemmArgs& a, hipStream_t s) {
  if (a.M <= 0 || a.N <= 0) return HI2X_OK;
  const dim3 grid((unsigned)((a.N + GT - 1) / GT), (unsigned)((a.M + GT - 1) / GT));
  hipLaunchKernelGGL((gemm_kernel<TB, ALOW, BLOW, CLOW>), grid, dim3(256), 0, s, a);
  return launch_status("gemm_kernel");
}

// ---- prep: P = J (hs + lam I) J, lam = damp * max(mean(diag hs), 1e-12) * 10^attempt ---
// mean(diag) as the reference's torch CPU reduction of the strided diagonal: 4 scalar
// accumulators over rows of 4, the 4-level cascade, the tail into accumulator 0, the
// accumulators folded, then divided by K.
__global__ void diag_mean_kernel(const float* __restrict__ hs, int64_t K, float damp,
                                 float p10, float* __restrict__ lam_out) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  auto x = [&](int64_t i) { return hs[i * K + i]; };
  const int64_t size_ilp = K / 4;
  float acc[4][4];
  for (int a = 0; a < 4; ++a)
    for (int b = 0; b < 4; ++b) acc[a][b] = 0.0f;
  if (size_ilp > 0) {
    int64_t lp = 1;
    if (size_ilp > 2) lp = 64 - __builtin_clzll((unsigned long long)(size_ilp - 1));
    lp /= 4;
    if (lp < 4) lp = 4;
    const int64_t step = (int64_t)1 << lp, lmask = step - 1;
    int64_t i = 0;
    while (i + step <= size_ilp) {
      for (int64_t j = 0; j < step; ++j)
        for (int q = 0; q < 4; ++q) acc[0][q] += x((i + j) * 4 + q);
      i += step;
      for (int lev = 1; lev < 4; ++lev) {
        for (int q = 0; q < 4; ++q) {
          acc[lev][q] += acc[lev - 1][q];
          acc[lev - 1][q] = 0.0f;
        }
        if (i & (lmask << (lev * lp))) break;
      }
    }
    for (; i < size_ilp; ++i)
      for (int q = 0; q < 4; ++q) acc[0][q] += x(i * 4 + q);
    for (int lev = 1; lev < 4; ++lev)
      for (int q = 0; q < 4; ++q) acc[0][q] += acc[lev][q];
  }
  float p[4] = {acc[0][0], acc[0][1], acc[0][2], acc[0][3]};
  for (int64_t i = size_ilp * 4; i < K; ++i) p[0] += x(i);
  const float sum = ((p[0] + p[1]) + p[2]) + p[3];
  float mean = sum / (float)K;
  mean = mean < 1e-12f ? 1e-12f : mean;
  *lam_out = (damp * mean) * p10;
}

__global__ __launch_bounds__(256) void reverse_damp_kernel(const float* __restrict__ hs,
                                                           int64_t K,
                                                           const float* __restrict__ lam,
                                                           float* __restrict__ P) {
  const int64_t i = (int64_t)blockIdx.y;
  const float l = *lam;
  for (int64_t j = threadIdx.x + (int64_t)blockIdx.x * blockDim.x; j <= i; j += (int64_t)gridDim.x * blockDim.x) {
    const float v = hs[(K - 1 - i) * K + (K - 1 - j)];
    P[i * K + j] = (i == j) ? v + l : v;
  }
}

// ---- diagonal block: factor in LDS, write L_jj, write inv(L_jj) to inv_out ----------
// status: first failing global pivot index + 1 (atomicMin over failures), 0 if none.
__global__ __launch_bounds__(256) void potrf_diag_kernel(float* __restrict__ P, int64_t K,
                                                         int64_t j0, int nb,
                                                         float* __restrict__ inv_out,
                                                         int* __restrict__ status) {
  __shared__ float T[NB][NB + 1];
  __shared__ float V[NB][NB + 1];
  const int tid = threadIdx.x;
  for (int idx = tid; idx < nb * nb; idx += 256) {
    const int i = idx / nb, j = idx % nb;
    T[i][j] = (j <= i) ? P[(j0 + i) * K + j0 + j] : 0.0f;
  }
  __syncthreads();
  for (int c = 0; c < nb; ++c) {
    if (tid == 0) {
      const float d = T[c][c];
      if (!(d > 0.0f)) {
        atomicMin(status, (int)(j0 + c + 1));
        T[c][c] = __builtin_nanf("");
      } else {
        T[c][c] = __builtin_sqrtf(d);
      }
    }
    __syncthreads();
    const float piv = T[c][c];
    for (int i = c + 1 + tid; i < nb; i += 256) T[i][c] = T[i][c] / piv;
    __syncthreads();
    const int m = nb - c - 1;
    for (int idx = tid; idx < m * m; idx += 256) {
      const int i = c + 1 + idx / m, j = c + 1 + idx % m;
      if (j <= i) T[i][j] = T[i][j] - T[i][c] * T[j][c];
    }
    __syncthreads();
  }
  for (int idx = tid; idx < nb * nb; idx += 256) {
    const int i = idx / nb, j = idx % nb;
    if (j <= i) P[(j0 + i) * K + j0 + j] = T[i][j];
  }
  // inverse of the lower triangular T, one column per thread (forward substitution)
  if (tid < nb) {
    const int j = tid;
    for (int i = 0; i < j; ++i) V[i][j] = 0.0f;
    V[j][j] = 1.0f / T[j][j];
    for (int i = j + 1; i < nb; ++i) {
      float s = 0.0f;
      for (int p = j; p < i; ++p) s = s + T[i][p] * V[p][j];
      V[i][j] = -s / T[i][i];
    }
  }
  __syncthreads();
  if (inv_out)
    for (int idx = tid; idx < nb * nb; idx += 256) {
      const int i = idx / nb, j = idx % nb;
      inv_out[(int64_t)i * NB + j] = V[i][j];
    }
}

// Copy an NB x NB inverse (ld NB) into the lower diagonal block of P at j0.
__global__ void put_diag_kernel(float* __restrict__ P, int64_t K, int64_t j0, int nb,
                                const float* __restrict__ inv) {
  for (int idx = threadIdx.x; idx < nb * nb; idx += blockDim.x) {
    const int i = idx / nb, j = idx % nb;
    if (j <= i) P[(j0 + i) * K + j0 + j] = inv[(int64_t)i * NB + j];
  }
}

// U[i][j] = Linv[K-1-i][K-1-j] for j >= i, 0 below: in place over pairs
// {(i, j), (K-1-i, K-1-j)}, thread per element of the upper triangle.
__global__ __launch_bounds__(256) void reverse_out_kernel(float* __restrict__ P, int64_t K) {
  const int64_t i = (int64_t)blockIdx.y;
  for (int64_t j = i + threadIdx.x + (int64_t)blockIdx.x * blockDim.x; j < K;
       j += (int64_t)gridDim.x * blockDim.x) {
    const int64_t ri = K - 1 - i, rj = K - 1 - j;  // (ri, rj) is in the lower triangle
    if (j == i) {
      if (i < ri) {
        const float a = P[i * K + i], b = P[ri * K + ri];
        P[i * K + i] = b;
        P[ri * K + ri] = a;
      }
    } else {
      P[i * K + j] = P[ri * K + rj];
      P[ri * K + rj] = 0.0f;
    }
  }
}

// ---- host driver --------------------------------------------------------------------
struct Chol {
  float* P;
  int64_t K;
  float* inv;   // [nblk, NB, NB] diagonal-block inverses
  float* tmp;   // [K/2 + NB, K/2 + NB] trtri temporary
  hipStream_t s;
};

int potrf(const Chol& c, int* status) {
  const int64_t K = c.K;
  for (int64_t j0 = 0; j0 < K; j0 += NB) {
    const int nb = (int)((K - j0 < NB) ? K - j0 : NB);
    float* inv = c.inv + (j0 / NB) * NB * NB;
    hipLaunchKernelGGL(potrf_diag_kernel, dim3(1), dim3(256), 0, c.s, c.P, K, j0, nb, inv,
                       status);
    int rc = launch_status("potrf_diag_kernel");
    if (rc) return rc;
    const int64_t m = K - j0 - nb;
    if (m <= 0) break;
    float* panel = c.P + (j0 + nb) * K + j0;
    // panel <- panel * inv(L_jj)^T   (in place: one column tile, rows read before written)
    GemmArgs a{panel, inv, panel, m, nb, nb, K, NB, K, 1.0f, 0.0f};
    rc = gemm<true, false, false, false>(a, c.s);
    if (rc) return rc;
    // trailing lower triangle: A22 -= panel * panel^T
    float* a22 = c.P + (j0 + nb) * K + (j0 + nb);
    GemmArgs b{panel, panel, a22, m, m, nb, K, K, K, -1.0f, 1.0f};
    rc = gemm<true, false, false, true>(b, c.s);
    if (rc) return rc;
  }
  return HI2X_OK;
}

// Lower triangular inverse of the diagonal region [r0, r0 + m) in place.
int trtri(const Chol& c, int64_t r0, int64_t m) {
  const int64_t K = c.K;
  if (m <= NB) {
    hipLaunchKernelGGL(put_diag_kernel, dim3(1), dim3(256), 0, c.s, c.P, K, r0, (int)m,
                       c.inv + (r0 / NB) * NB * NB);
    return launch_status("put_diag_kernel");
  }
  const int64_t nbk = (m + NB - 1) / NB;
  const int64_t m1 = ((nbk + 1) / 2) * NB, m2 = m - m1;
  int rc = trtri(c, r0, m1);
  if (rc) return rc;
  rc = trtri(c, r0 + m1, m2);
  if (rc) return rc;
  float* Ainv = c.P + r0 * K + r0;               // m1 x m1, lower
  float* Bblk = c.P + (r0 + m1) * K + r0;        // m2 x m1, full (original L)
  float* Cinv = c.P + (r0 + m1) * K + (r0 + m1); // m2 x m2, lower
  // tmp = B * A^-1   (op(B) = A^-1 lower: k >= j)
  GemmArgs g1{Bblk, Ainv, c.tmp, m2, m1, m1, K, K, m1, 1.0f, 0.0f};
  rc = gemm<false, false, true, false>(g1, c.s);
  if (rc) return rc;
  // B <- -C^-1 * tmp  (A = C^-1 lower: k <= i)
  GemmArgs g2{Cinv, c.tmp, Bblk, m2, m1, m2, K, m1, K, -1.0f, 0.0f};
  return gemm<false, true, false, false>(g2, c.s);
}

}  // namespace
}  // namespace hi2x

using namespace hi2x;

extern "C" int hi2x_chol_inv_upper(const float* hs, int64_t k, float damp, int attempt,
                                   float* u, void* stream) {
  clear_error();
  HI2X_REQUIRE(k > 0 && hs && u && hs != u, "chol_inv_upper: bad arguments");
  HI2X_REQUIRE(attempt >= 0 && attempt < 10, "chol_inv_upper: attempt %d", attempt);
  hipStream_t s = as_stream(stream);
  const int64_t nblk = (k + NB - 1) / NB;
  const int64_t half = (nblk + 1) / 2 * NB;
  float* inv = nullptr;
  float* tmp = nullptr;
  int* status = nullptr;
  float* lam = nullptr;
  const size_t inv_bytes = (size_t)nblk * NB * NB * sizeof(float);
  const size_t tmp_bytes = (size_t)half * (size_t)half * sizeof(float);
  HI2X_HIP(hipMallocAsync((void**)&inv, inv_bytes, s));
  HI2X_HIP(hipMallocAsync((void**)&tmp, tmp_bytes, s));
  HI2X_HIP(hipMallocAsync((void**)&status, 2 * sizeof(int) + sizeof(float), s));
  lam = reinterpret_cast<float*>(status + 2);
  const int big = 0x7fffffff;
  HI2X_HIP(hipMemcpyAsync(status, &big, sizeof(int), hipMemcpyHostToDevice, s));
  float p10 = 1.0f;
  for (int a = 0; a < attempt; ++a) p10 *= 10.0f;
  hipLaunchKernelGGL(diag_mean_kernel, dim3(1), dim3(64), 0, s, hs, k, damp, p10, lam);
  int rc = launch_status("diag_mean_kernel");
  if (!rc) {
    const dim3 g((unsigned)((k + 255) / 256 < 16 ? (k + 255) / 256 : 16), (unsigned)k);
    hipLaunchKernelGGL(reverse_damp_kernel, g, dim3(256), 0, s, hs, k, lam, u);
    rc = launch_status("reverse_damp_kernel");
  }
  Chol c{u, k, inv, tmp, s};
  if (!rc) rc = potrf(c, status);
  int st = big;
  if (!rc) {
    hipError_t e = hipMemcpyAsync(&st, status, sizeof(int), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) {
      set_error("chol_inv_upper: status read: %s", hipGetErrorString(e));
      rc = HI2X_ELAUNCH;
    }
  }
  if (!rc && st != big) {
    set_error("chol_inv_upper: not positive definite at pivot %d (attempt %d)", st - 1, attempt);
    rc = HI2X_ENOTPD;
  }
  if (!rc) rc = trtri(c, 0, k);
  if (!rc) {
    const dim3 g((unsigned)((k + 255) / 256 < 16 ? (k + 255) / 256 : 16), (unsigned)k);
    hipLaunchKernelGGL(reverse_out_kernel, g, dim3(256), 0, s, u, k);
    rc = launch_status("reverse_out_kernel");
  }
  (void)hipFreeAsync(inv, s);
  (void)hipFreeAsync(tmp, s);
  (void)hipFreeAsync(status, s);
  return rc;
}
