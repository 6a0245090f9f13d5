// Eigen-decomposition of the closure scatter (the first-call basis).
//   symmetric_eigen   eigenvalues and eigenvectors of 0.5 (A + A^T) for a batch of small
//                     fp32 matrices (n <= 128), eigenvalues ascending and eigenvectors as
//                     columns, the contract of torch.linalg.eigh that closure_basis calls
//                     (recap/sparse/closure.py:75-81).
//
// One workgroup per matrix; the matrix and the accumulated rotations live in LDS (2 x 64 KB
// at n = 128).  Two-sided cyclic Jacobi (Golub & Van Loan, Matrix Computations, 4th ed.,
// alg. 8.5.2 with the symmetric 2x2 Schur rotation of alg. 8.5.1) in the parallel
// round-robin ordering of Brent & Luk (1985): a sweep is m - 1 rounds (m = n rounded up
// to even) of m/2 disjoint index pairs, rotated at once.  A round is two barriers: the m/2
// threads that own a pair compute its rotation and publish it with the pair, then every
// thread applies J_k^T B J_l to whole 2x2 blocks (k, l) of the matrix, so the row and
// column passes need no barrier between them, and V <- V J to the rotation matrix.
//
// Off-diagonal entries are only ever formed from off-diagonal entries, so the rounding
// noise they carry shrinks with them and the relative test of Demmel & Veselic (1992),
// |a_pq| <= tol sqrt(|a_pp a_qq|), is reached; a sweep that rotates nothing ends the loop,
// and a fixed sweep cap bounds it whatever the input.
#include "kernels.hpp"

namespace recap {

namespace {

constexpr int kEigenMax = 128;
constexpr int kEigenThreads = 1024;    // 4 waves per SIMD hide the LDS latency of a round
constexpr float kEigenTol = 1.0e-7f;   // ~ 2 fp32 ulps of 1

// Pair k of round r in the circle ordering of m (even) indices: every unordered pair once
// per sweep of m - 1 rounds.
__device__ __forceinline__ void round_pair(int m, int r, int k, int& p, int& q) {
  if (k == 0) { p = m - 1; q = r; return; }
  const int c = m - 1;
  p = r + k; if (p >= c) p -= c;
  q = r - k; if (q < 0) q += c;
}

__global__ __launch_bounds__(kEigenThreads) void symmetric_eigen_kernel(EigenArgs a) {
  __shared__ __attribute__((aligned(16))) float A[kEigenMax * kEigenMax];
  __shared__ __attribute__((aligned(16))) float V[kEigenMax * kEigenMax];
  __shared__ float rot_c[kEigenMax / 2], rot_s[kEigenMax / 2];
  __shared__ int pair_p[kEigenMax / 2], pair_q[kEigenMax / 2];
  __shared__ float lam[kEigenMax];
  __shared__ int rank[kEigenMax];
  __shared__ int rotated;
  const int t = threadIdx.x, n = a.n, m = a.m, half = m / 2;
  // Fixed work map of a round: pair column l = t % 64 for every block (k, l) and rotation
  // column of this thread, pair rows k = t / 64 + 16 j (blocks) and V rows i = t / 64 + 16 j.
  const int l = t & 63, k0 = t >> 6;
  const float* src = a.a + (int64_t)blockIdx.x * n * n;

  // The whole 128 x 128 storage is defined (zero outside n x n, V = I) so the tiled
  // products below may read past n.
  for (int idx = t; idx < kEigenMax * kEigenMax; idx += kEigenThreads) {
    const int i = idx >> 7, j = idx & (kEigenMax - 1);
    float x = 0.0f;
    if (i < n && j < n) x = 0.5f * (src[i * n + j] + src[j * n + i]);
    A[idx] = x;
    V[idx] = (i == j) ? 1.0f : 0.0f;
  }
  if (t == 0) rotated = 0;
  __syncthreads();

  for (int sweep = 0; sweep < a.max_sweeps; ++sweep) {
    for (int r = 0; r < m - 1; ++r) {
      if (t < half) {
        int p, q;
        round_pair(m, r, t, p, q);
        const float app = A[p * kEigenMax + p], aqq = A[q * kEigenMax + q];
        const float apq = A[p * kEigenMax + q];
        float c = 1.0f, s = 0.0f;
        if (fabsf(apq) > kEigenTol * sqrtf(fabsf(app * aqq)) && apq != 0.0f) {
          // t = tan(theta) of the smaller rotation that zeroes a_pq (alg. 8.5.1).
          const float tau = (aqq - app) / (2.0f * apq);
          const float tn = copysignf(1.0f, tau) / (fabsf(tau) + sqrtf(1.0f + tau * tau));
          c = 1.0f / sqrtf(1.0f + tn * tn);
          s = tn * c;
          rotated = 1;
        }
        rot_c[t] = c; rot_s[t] = s;
        pair_p[t] = p; pair_q[t] = q;
      }
      __syncthreads();
      if (l < half) {
        const int pl = pair_p[l], ql = pair_q[l];
        const float cl = rot_c[l], sl = rot_s[l];
        // B <- J^T B J over 2x2 blocks: rows (p_k, q_k), columns (p_l, q_l).
#pragma unroll
        for (int j = 0; j < kEigenMax / 2 / (kEigenThreads / 64); ++j) {
          const int k = k0 + (kEigenThreads / 64) * j;
          if (k >= half) break;
          const int pk = pair_p[k], qk = pair_q[k];
          const float ck = rot_c[k], sk = rot_s[k];
          if (k == l) {
            // Diagonal block: the closed form, with the zeroed entry set exactly.
            const float apq = A[pk * kEigenMax + qk];
            const float tn = (ck != 0.0f) ? sk / ck : 0.0f;
            A[pk * kEigenMax + pk] -= tn * apq;
            A[qk * kEigenMax + qk] += tn * apq;
            if (sk != 0.0f) { A[pk * kEigenMax + qk] = 0.0f; A[qk * kEigenMax + pk] = 0.0f; }
            continue;
          }
          const float b_pp = A[pk * kEigenMax + pl], b_pq = A[pk * kEigenMax + ql];
          const float b_qp = A[qk * kEigenMax + pl], b_qq = A[qk * kEigenMax + ql];
          // rows: r_p = c_k b_p - s_k b_q, r_q = s_k b_p + c_k b_q
          const float r_pp = ck * b_pp - sk * b_qp, r_pq = ck * b_pq - sk * b_qq;
          const float r_qp = sk * b_pp + ck * b_qp, r_qq = sk * b_pq + ck * b_qq;
          // columns: x_p = c_l r_p - s_l r_q, x_q = s_l r_p + c_l r_q
          A[pk * kEigenMax + pl] = cl * r_pp - sl * r_pq;
          A[pk * kEigenMax + ql] = sl * r_pp + cl * r_pq;
          A[qk * kEigenMax + pl] = cl * r_qp - sl * r_qq;
          A[qk * kEigenMax + ql] = sl * r_qp + cl * r_qq;
        }
        // V <- V J: columns (p_l, q_l) of rows i.
#pragma unroll
        for (int j = 0; j < kEigenMax / (kEigenThreads / 64); ++j) {
          const int i = k0 + (kEigenThreads / 64) * j;
          if (i >= m) break;
          const float vp = V[i * kEigenMax + pl], vq = V[i * kEigenMax + ql];
          V[i * kEigenMax + pl] = cl * vp - sl * vq;
          V[i * kEigenMax + ql] = sl * vp + cl * vq;
        }
      }
      __syncthreads();
    }
    const int any = rotated;   // read by every thread after the round's last barrier
    __syncthreads();
    if (t == 0) rotated = 0;
    __syncthreads();
    if (!any) break;
  }

  // One Newton-Schulz step towards the nearest orthogonal matrix, V <- V (3I - V^T V) / 2,
  // removes the rounding drift the sweeps of rotations leave in V's orthogonality (~1e-5
  // at n = 128, down to ~1e-6) without moving it off the eigenvectors.
  for (int i = t; i < n; i += kEigenThreads) lam[i] = A[i * kEigenMax + i];
  __syncthreads();
  const int n4 = (n + 3) / 4;
  for (int tile = t; tile < n4 * n4; tile += kEigenThreads) {
    const int i0 = 4 * (tile / n4), j0 = 4 * (tile % n4);
    float e[4][4] = {};
    for (int r = 0; r < n; ++r) {
      const float4 vi = *reinterpret_cast<const float4*>(&V[r * kEigenMax + i0]);
      const float4 vj = *reinterpret_cast<const float4*>(&V[r * kEigenMax + j0]);
      const float xi[4] = {vi.x, vi.y, vi.z, vi.w}, xj[4] = {vj.x, vj.y, vj.z, vj.w};
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int w = 0; w < 4; ++w) e[u][w] = fmaf(xi[u], xj[w], e[u][w]);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int w = 0; w < 4; ++w)
        A[(i0 + u) * kEigenMax + j0 + w] = e[u][w] - ((i0 + u == j0 + w) ? 1.0f : 0.0f);
  }
  __syncthreads();
  {
    // Eight threads per row, 16 columns each: row i of V (E) accumulated, then written back
    // after every thread has finished reading V.
    const int i = t >> 3, j0 = 16 * (t & 7);
    float acc[16];
#pragma unroll
    for (int w = 0; w < 16; ++w) acc[w] = 0.0f;
    if (i < n) {
      for (int r = 0; r < n; ++r) {
        const float v = V[i * kEigenMax + r];
#pragma unroll
        for (int w = 0; w < 16; ++w) acc[w] = fmaf(v, A[r * kEigenMax + j0 + w], acc[w]);
      }
    }
    __syncthreads();
    if (i < n) {
#pragma unroll
      for (int w = 0; w < 16; ++w)
        if (j0 + w < n) V[i * kEigenMax + j0 + w] -= 0.5f * acc[w];
    }
  }

  // Ascending order of the n real eigenvalues, ties to the lower index (the padded index
  // n, when n is odd, is an isolated zero row and is dropped).
  for (int i = t; i < n; i += kEigenThreads) {
    const float li = lam[i];
    int rk = 0;
    for (int j = 0; j < n; ++j) {
      const float lj = lam[j];
      rk += (lj < li) || (lj == li && j < i);
    }
    rank[i] = rk;
    a.values[(int64_t)blockIdx.x * n + rk] = li;
  }
  __syncthreads();
  float* dst = a.vectors + (int64_t)blockIdx.x * n * n;
  for (int idx = t; idx < n * n; idx += kEigenThreads) {
    const int i = idx / n, j = idx % n;
    dst[i * n + rank[j]] = V[i * kEigenMax + j];
  }
}

}  // namespace

hipError_t run_symmetric_eigen(const EigenArgs& a, hipStream_t s) {
  if (a.n < 1 || a.n > kEigenMax || a.m != a.n + (a.n & 1) || a.batch < 1)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(symmetric_eigen_kernel, dim3(a.batch), dim3(kEigenThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace recap
