// Device-side kernel templates of the MI355X backend, prepended to every
// hipRTC program.  The code generator supplies small functors (operand
// loaders with the access expression inlined, and an epilogue with the fused
// elementwise statements) and instantiates one of the templates below.
//
//  * dp_mfma      -- DotProd+Elw: fp32 MFMA (v_mfma_f32_32x32x2_f32), 128x128
//                    block tile, 4 waves of 64x64, LDS-staged K panels with a
//                    register prefetch of the next panel, epilogue in registers.
//  * reduce_rows  -- Reduce+Elw, rows contiguous: one wave per row, float4 or
//                    scalar coalesced loads, butterfly over the wave.
//  * reduce_cols  -- Reduce+Elw, columns contiguous: 64 columns x 4 row groups
//                    per block, coalesced along the columns, LDS combine.
// Elementwise (ElwFuse) kernels are emitted whole by the generator.
#pragma clang fp contract(off)

typedef float adhip_f32x16 __attribute__((ext_vector_type(16)));

namespace adhip {

template <int OP>
__device__ __forceinline__ float rop(float a, float b) {
  if constexpr (OP == 0) return a + b;
  else return fmaxf(a, b);
}

// ---------------------------------------------------------------- DotProd+Elw
// LA::at(m, k), LB::at(k, n) load one element (no bounds check);
// LA::at4 / LB::at4 load 4 consecutive elements along the contiguous axis.
// LA::kMode: 0 = contiguous along k, 1 = contiguous along m.
// LB::kMode: 0 = contiguous along n, 1 = contiguous along k.
constexpr int DP_BM = 128, DP_BN = 128, DP_BK = 16, DP_PAD = 4;

template <class LA, class LB, class EPI>
__device__ __forceinline__ void dp_mfma(const LA& la, const LB& lb, const EPI& epi, int M, int N, int K) {
  __shared__ float As[DP_BK][DP_BM + DP_PAD];
  __shared__ float Bs[DP_BK][DP_BN + DP_PAD];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * DP_BM, n0 = blockIdx.x * DP_BN;

  float ra[8], rb[8];

  auto load_a = [&](int k0) {
    if constexpr (LA::kMode == 0) {            // thread: one row, 8 consecutive k
      const int m = m0 + (tid >> 1);
      const int kb = k0 + (tid & 1) * 8;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int k = kb + 4 * h;
        if constexpr (LA::kVec) {
          float4 v = (m < M && k < K) ? la.at4(m, k) : make_float4(0.f, 0.f, 0.f, 0.f);
          ra[4 * h + 0] = v.x; ra[4 * h + 1] = v.y; ra[4 * h + 2] = v.z; ra[4 * h + 3] = v.w;
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) ra[4 * h + j] = (m < M && k + j < K) ? la.at(m, k + j) : 0.f;
        }
      }
    } else {                                    // thread: one k, 8 consecutive rows
      const int k = k0 + (tid >> 4);
      const int mb = m0 + (tid & 15) * 8;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int m = mb + 4 * h;
        if constexpr (LA::kVec) {
          float4 v = (k < K && m < M) ? la.at4(m, k) : make_float4(0.f, 0.f, 0.f, 0.f);
          ra[4 * h + 0] = v.x; ra[4 * h + 1] = v.y; ra[4 * h + 2] = v.z; ra[4 * h + 3] = v.w;
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) ra[4 * h + j] = (k < K && m + j < M) ? la.at(m + j, k) : 0.f;
        }
      }
    }
  };
  auto store_a = [&]() {
    if constexpr (LA::kMode == 0) {
      const int m = tid >> 1, kb = (tid & 1) * 8;
#pragma unroll
      for (int j = 0; j < 8; ++j) As[kb + j][m] = ra[j];
    } else {
      const int k = tid >> 4, mb = (tid & 15) * 8;
      *reinterpret_cast<float4*>(&As[k][mb]) = make_float4(ra[0], ra[1], ra[2], ra[3]);
      *reinterpret_cast<float4*>(&As[k][mb + 4]) = make_float4(ra[4], ra[5], ra[6], ra[7]);
    }
  };
  auto load_b = [&](int k0) {
    if constexpr (LB::kMode == 0) {            // thread: one k, 8 consecutive n
      const int k = k0 + (tid >> 4);
      const int nb = n0 + (tid & 15) * 8;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int n = nb + 4 * h;
        if constexpr (LB::kVec) {
          float4 v = (k < K && n < N) ? lb.at4(k, n) : make_float4(0.f, 0.f, 0.f, 0.f);
          rb[4 * h + 0] = v.x; rb[4 * h + 1] = v.y; rb[4 * h + 2] = v.z; rb[4 * h + 3] = v.w;
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) rb[4 * h + j] = (k < K && n + j < N) ? lb.at(k, n + j) : 0.f;
        }
      }
    } else {                                    // thread: one n, 8 consecutive k
      const int n = n0 + (tid >> 1);
      const int kb = k0 + (tid & 1) * 8;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int k = kb + 4 * h;
        if constexpr (LB::kVec) {
          float4 v = (n < N && k < K) ? lb.at4(k, n) : make_float4(0.f, 0.f, 0.f, 0.f);
          rb[4 * h + 0] = v.x; rb[4 * h + 1] = v.y; rb[4 * h + 2] = v.z; rb[4 * h + 3] = v.w;
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) rb[4 * h + j] = (n < N && k + j < K) ? lb.at(k + j, n) : 0.f;
        }
      }
    }
  };
  auto store_b = [&]() {
    if constexpr (LB::kMode == 0) {
      const int k = tid >> 4, nb = (tid & 15) * 8;
      *reinterpret_cast<float4*>(&Bs[k][nb]) = make_float4(rb[0], rb[1], rb[2], rb[3]);
      *reinterpret_cast<float4*>(&Bs[k][nb + 4]) = make_float4(rb[4], rb[5], rb[6], rb[7]);
    } else {
      const int n = tid >> 1, kb = (tid & 1) * 8;
#pragma unroll
      for (int j = 0; j < 8; ++j) Bs[kb + j][n] = rb[j];
    }
  };

  adhip_f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  load_a(0);
  load_b(0);
  store_a();
  store_b();
  __syncthreads();
  const int lk = lane >> 5, lr = lane & 31;
  for (int k0 = 0; k0 < K; k0 += DP_BK) {
    const bool more = k0 + DP_BK < K;
    if (more) {
      load_a(k0 + DP_BK);
      load_b(k0 + DP_BK);
    }
#pragma unroll
    for (int kk = 0; kk < DP_BK; kk += 2) {
      const float a0 = As[kk + lk][wm * 64 + lr];
      const float a1 = As[kk + lk][wm * 64 + 32 + lr];
      const float b0 = Bs[kk + lk][wn * 64 + lr];
      const float b1 = Bs[kk + lk][wn * 64 + 32 + lr];
      acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b0, acc[0][0], 0, 0, 0);
      acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b1, acc[0][1], 0, 0, 0);
      acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b0, acc[1][0], 0, 0, 0);
      acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b1, acc[1][1], 0, 0, 0);
    }
    __syncthreads();
    if (more) {
      store_a();
      store_b();
      __syncthreads();
    }
  }
  // 32x32 accumulator layout: lane holds column (lane % 32) and rows
  // 8*(r/4) + 4*(lane/32) + r%4 for r = 0..15
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
        const int col = n0 + wn * 64 + j * 32 + lr;
        if (row < M && col < N) epi(acc[i][j][r], row, col);
      }
}

// ---------------------------------------------------------------- Reduce+Elw
// LD::at(x, y) loads element y of reduced row x; LD::at4 four consecutive y.
// LD::inc(y) is false for elements the reference's work-group tree drops.
template <int OP, class LD, class EPI>
__device__ __forceinline__ void reduce_rows(const LD& ld, const EPI& epi, unsigned V, unsigned R,
                                            bool pad_zero) {
  const unsigned lane = threadIdx.x & 63;
  const unsigned row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= V) return;
  float acc = OP == 0 ? 0.f : -__builtin_huge_valf();
  if constexpr (LD::kVec) {
    float acc2 = acc;
    unsigned y = lane * 4;
    for (; y + 256 < R; y += 512) {
      const float4 v = ld.at4(row, y);
      const float4 w = ld.at4(row, y + 256);
      acc = rop<OP>(rop<OP>(acc, v.x), v.y);
      acc2 = rop<OP>(rop<OP>(acc2, v.z), v.w);
      acc = rop<OP>(rop<OP>(acc, w.x), w.y);
      acc2 = rop<OP>(rop<OP>(acc2, w.z), w.w);
    }
    if (y < R) {
      const float4 v = ld.at4(row, y);
      acc = rop<OP>(rop<OP>(acc, v.x), v.y);
      acc2 = rop<OP>(rop<OP>(acc2, v.z), v.w);
    }
    acc = rop<OP>(acc, acc2);
  } else {
    for (unsigned y = lane; y < R; y += 64)
      if (ld.inc(y)) acc = rop<OP>(acc, ld.at(row, y));
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) acc = rop<OP>(acc, __shfl_xor(acc, off, 64));
  if (OP == 1 && pad_zero) acc = fmaxf(acc, 0.f);
  if (lane == 0) epi(acc, row);
}

template <int OP, class LD, class EPI>
__device__ __forceinline__ void reduce_cols(const LD& ld, const EPI& epi, unsigned V, unsigned R,
                                            bool pad_zero) {
  __shared__ float part[4][64];
  const unsigned lane = threadIdx.x & 63, grp = threadIdx.x >> 6;
  const unsigned col = blockIdx.x * 64 + lane;
  float acc = OP == 0 ? 0.f : -__builtin_huge_valf();
  if (col < V)
    for (unsigned y = grp; y < R; y += 4)
      if (ld.inc(y)) acc = rop<OP>(acc, ld.at(col, y));
  part[grp][lane] = acc;
  __syncthreads();
  if (grp == 0 && col < V) {
    acc = rop<OP>(rop<OP>(rop<OP>(part[0][lane], part[1][lane]), part[2][lane]), part[3][lane]);
    if (OP == 1 && pad_zero) acc = fmaxf(acc, 0.f);
    epi(acc, col);
  }
}

}  // namespace adhip
