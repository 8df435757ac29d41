// Device-side kernel templates of the MI355X backend, prepended to every
// hipRTC program.  The code generator supplies small functors (operand
// loaders with the access expression inlined, and an epilogue with the fused
// elementwise statements) and instantiates one of the templates below.
//
//  * dp_mfma      -- DotProd+Elw: fp32 MFMA (v_mfma_f32_32x32x2_f32), BM x BN
//                    block tile (64..256), 4 waves, LDS-staged K panels with a
//                    register prefetch of the next panel, optional split of K
//                    into chunks, epilogue in registers.
//  * dp_quad      -- the same on 32 x 32 tiles with each block's K panels
//                    split among its 4 waves, for launches too small to
//                    fill the device.
//  * reduce_rows  -- Reduce+Elw, rows contiguous: waves striding over rows,
//                    float4 or scalar coalesced loads, butterfly over the wave.
//  * reduce_cols  -- Reduce+Elw, columns contiguous: 64 columns x 4 or 16
//                    (float4 lanes) row groups per block, coalesced along
//                    the columns, LDS combine, optional split of the rows.
//  * pack_bf16, dp_bf16 -- the bf16 DotProd option: operands packed as
//                    k-contiguous bf16, v_mfma_f32_32x32x16_bf16, fp32 sums.
// Elementwise (ElwFuse) kernels are emitted whole by the generator.
#pragma clang fp contract(off)

typedef float adhip_f32x16 __attribute__((ext_vector_type(16)));
typedef float adhip_f32x4 __attribute__((ext_vector_type(4)));

namespace adhip {

// float4 load / store of generated code; S = true streams the data
// (nontemporal: the lines are not kept in the caches), for operands too
// large for the caches to hold until anyone reads them again.
template <bool S>
__device__ __forceinline__ float4 ld4(const float* p) {
  if constexpr (S) {
    const adhip_f32x4 t = __builtin_nontemporal_load(reinterpret_cast<const adhip_f32x4*>(p));
    return make_float4(t.x, t.y, t.z, t.w);
  } else {
    return *reinterpret_cast<const float4*>(p);
  }
}

template <bool S>
__device__ __forceinline__ void st4(float* p, float4 v) {
  if constexpr (S) {
    const adhip_f32x4 t = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(t, reinterpret_cast<adhip_f32x4*>(p));
  } else {
    *reinterpret_cast<float4*>(p) = v;
  }
}

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
//
// Block tile BM x BN, K panels of BK staged in two LDS buffers, 4 waves as
// 2 x 2, each wave (BM/2) x (BN/2) made of 32x32 v_mfma_f32_32x32x2f32 tiles;
// the next panel is prefetched into registers while the current one is
// consumed, then stored into the other buffer.  A lane reads its operand
// fragments for 4 MFMA steps at a time (one float4 per 32-row tile for an
// operand kept k-contiguous in LDS).
// SPLIT > 1 splits K into SPLIT chunks: blockIdx.y = tile row + tiles_m *
// chunk, and the epilogue receives the chunk index (partial results).
// Epilogue, EPI::kVec4 false: per 32x32 tile, epi.load(row, col, l) fills
// the operand registers l[EPI::kLoads] of all 16 values of a lane, then
// epi(value, row, col, chunk, l) runs the statements of each.
// EPI::kVec4 true (N a multiple of 4): each wave passes its 32x32 tiles
// through LDS so a lane holds 4 consecutive columns of a row; per tile,
// epi.load4(row, col, l) fills float4 operand registers for the lane's 4
// groups, then epi.vec(value4, row, col, chunk, l) runs the statements on 4
// elements with float4 loads and stores.
constexpr int DP_GROUP = 8, DP_CPITCH = 40;

// Block -> output tile.  Workgroups go to the 8 XCDs round-robin, each XCD
// with its own L2: give every XCD a contiguous run of tiles, ordered in
// groups of DP_GROUP tile rows, so blocks sharing A rows and B columns share
// an L2.
__device__ __forceinline__ void dp_block_tile(int& bx, int& by) {
  const int gx = gridDim.x, gy = gridDim.y, T = gx * gy;
  int L = blockIdx.y * gx + blockIdx.x;
  if (T % 8 == 0) L = (L % 8) * (T / 8) + L / 8;
  const int per_group = DP_GROUP * gx;
  const int first = (L / per_group) * DP_GROUP;
  const int rows = gy - first < DP_GROUP ? gy - first : DP_GROUP;
  by = first + (L % per_group) % rows;
  bx = (L % per_group) / rows;
}

// Epilogue of a DotProd block: the 32x32 accumulator tiles of each wave go
// through EPI (see the DotProd+Elw notes above); `smem` is the block's LDS,
// free once the products are done (at least 4 * 32 * DP_CPITCH floats).
template <int BM, int BN, class EPI>
__device__ __forceinline__ void dp_epilogue(const EPI& epi, adhip_f32x16 (&acc)[BM / 64][BN / 64], float* smem,
                                            int m0, int n0, int M, int N, int chunk) {
  constexpr int TM = BM / 64, TN = BN / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int lk = lane >> 5, lr = lane & 31;
  // 32x32 accumulator layout: lane holds column (lane % 32) and rows
  // 8*(r/4) + 4*(lane/32) + r%4 for r = 0..15.  Per 32x32 tile, the
  // epilogue's operand loads for all 16 values are issued first, then the
  // statements run.
  constexpr int NL = EPI::kLoads > 0 ? EPI::kLoads : 1;
  if constexpr (EPI::kVec4) {
    // lane -> row 8*q + lane/8 and columns 4*(lane%8) .. +3 of the tile
    __syncthreads();
    float* cs = smem + wave * 32 * DP_CPITCH;
    const int qr = lane >> 3, qc = 4 * (lane & 7);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int col = n0 + wn * (BN / 2) + j * 32 + qc;
        const int rbase = m0 + wm * (BM / 2) + i * 32 + qr;
        float4 lv[4][NL];
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (rbase + 8 * q < M && col < N) epi.load4(rbase + 8 * q, col, lv[q]);
#pragma unroll
        for (int r = 0; r < 16; ++r) cs[(8 * (r >> 2) + 4 * lk + (r & 3)) * DP_CPITCH + lr] = acc[i][j][r];
        // lanes read what other lanes of the wave wrote (LDS executes a
        // wave's operations in order; the fences keep the compiler's order)
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        float4 v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = *reinterpret_cast<const float4*>(cs + (8 * q + qr) * DP_CPITCH + qc);
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (rbase + 8 * q < M && col < N) epi.vec(v[q], rbase + 8 * q, col, chunk, lv[q]);
      }
  } else {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        float lv[16][NL];
        const int col = n0 + wn * (BN / 2) + j * 32 + lr;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = m0 + wm * (BM / 2) + i * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
          if (row < M && col < N) epi.load(row, col, lv[r]);
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = m0 + wm * (BM / 2) + i * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
          if (row < M && col < N) epi(acc[i][j][r], row, col, chunk, lv[r]);
        }
      }
  }
}

template <int BM, int BN, int SPLIT, int BK, class LA, class LB, class EPI, int NBUF = 2>
__device__ __forceinline__ void dp_mfma(const LA& la, const LB& lb, const EPI& epi, int M, int N, int K) {
  static_assert(NBUF == 1 || NBUF == 2, "one or two LDS panel buffers");
  static_assert(BM % 64 == 0 && BN % 64 == 0, "tile must be a multiple of 64");
  static_assert(BK % 16 == 0, "K panel must be a multiple of 16");
  constexpr int TM = BM / 64, TN = BN / 64;              // 32x32 tiles per wave
  constexpr int VA = BM * BK / 4 / 256;               // float4 loads per thread
  constexpr int VB = BN * BK / 4 / 256;
  static_assert(VA >= 1 && VB >= 1, "tile too small for 256 threads");
  // LDS layout of a K panel: an operand contiguous along k in memory (A
  // kMode 0, B kMode 1) is kept as [row][k] (pitch KP = BK + 4 floats), so a
  // lane reads the 4 consecutive k of 4 MFMA steps as one float4; the other
  // as [k][row] (pitch rows + 4), read as scalars.  Panel loads and stores
  // are float4s along the contiguous axis.  (Transposing the second operand
  // into [row][k] too needs k-fastest lanes for conflict-free stores, which
  // breaks the coalescing of its loads: measured slower.)
  // K panels (two buffers of A and of B) and, after the products, the
  // per-wave 32x32 staging of the vectorised epilogue share one LDS block.
  constexpr bool AR = LA::kMode == 0, BR = LB::kMode == 1;
  constexpr int KP = BK + 4, H = BK / 2;
  constexpr int APITCH = AR ? KP : BM + 4, BPITCH = BR ? KP : BN + 4;
  constexpr int A_FLOATS = NBUF * (AR ? BM : BK) * APITCH, B_FLOATS = NBUF * (BR ? BN : BK) * BPITCH;
  constexpr int C_FLOATS = EPI::kVec4 ? 4 * 32 * DP_CPITCH : 0;
  constexpr int S_FLOATS = A_FLOATS + B_FLOATS > C_FLOATS ? A_FLOATS + B_FLOATS : C_FLOATS;
  __shared__ __attribute__((aligned(16))) float smem[S_FLOATS];
  float* const As = smem;
  float* const Bs = smem + A_FLOATS;
  // float offset of element (row, k) of panel buffer `buf`
  auto a_off = [](int buf, int m, int k) { return AR ? (buf * BM + m) * APITCH + k : (buf * BK + k) * APITCH + m; };
  auto b_off = [](int buf, int n, int k) { return BR ? (buf * BN + n) * BPITCH + k : (buf * BK + k) * BPITCH + n; };
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int tiles_m = (M + BM - 1) / BM;
  int bx, by;
  dp_block_tile(bx, by);
  const int chunk = SPLIT > 1 ? by / tiles_m : 0;
  const int m0 = (SPLIT > 1 ? by % tiles_m : by) * BM, n0 = bx * BN;
  int kbeg = 0, kend = K;
  if constexpr (SPLIT > 1) {
    const int kc = ((K + SPLIT - 1) / SPLIT + BK - 1) / BK * BK;
    kbeg = chunk * kc;
    kend = kbeg + kc < K ? kbeg + kc : K;
  }

  float ra[VA][4], rb[VB][4];

  // float4 v of a panel (v < rows * BK / 4): (row, k) of its first float
  auto a_pos = [](int v, int& m, int& k) {
    if constexpr (AR) { m = v / (BK / 4); k = 4 * (v % (BK / 4)); }
    else { k = v / (BM / 4); m = 4 * (v % (BM / 4)); }
  };
  auto b_pos = [](int v, int& n, int& k) {
    if constexpr (BR) { n = v / (BK / 4); k = 4 * (v % (BK / 4)); }
    else { k = v / (BN / 4); n = 4 * (v % (BN / 4)); }
  };
  auto load_a = [&](int k0) {
#pragma unroll
    for (int i = 0; i < VA; ++i) {
      int m, k;
      a_pos(tid + 256 * i, m, k);
      m += m0;
      k += k0;
      if constexpr (LA::kMode == 0) {          // 4 consecutive k of row m
        if constexpr (LA::kVec) {
          const float4 x = (m < M && k < kend) ? la.at4(m, k) : make_float4(0.f, 0.f, 0.f, 0.f);
          ra[i][0] = x.x; ra[i][1] = x.y; ra[i][2] = x.z; ra[i][3] = x.w;
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) ra[i][j] = (m < M && k + j < kend) ? la.at(m, k + j) : 0.f;
        }
      } else {                                  // 4 consecutive m of k row
        if constexpr (LA::kVec) {
          const float4 x = (k < kend && m < M) ? la.at4(m, k) : make_float4(0.f, 0.f, 0.f, 0.f);
          ra[i][0] = x.x; ra[i][1] = x.y; ra[i][2] = x.z; ra[i][3] = x.w;
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) ra[i][j] = (k < kend && m + j < M) ? la.at(m + j, k) : 0.f;
        }
      }
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < VA; ++i) {
      int m, k;
      a_pos(tid + 256 * i, m, k);
      *reinterpret_cast<float4*>(As + a_off(buf, m, k)) = make_float4(ra[i][0], ra[i][1], ra[i][2], ra[i][3]);
    }
  };
  auto load_b = [&](int k0) {
#pragma unroll
    for (int i = 0; i < VB; ++i) {
      int n, k;
      b_pos(tid + 256 * i, n, k);
      n += n0;
      k += k0;
      if constexpr (LB::kMode == 0) {          // 4 consecutive n of k row
        if constexpr (LB::kVec) {
          const float4 x = (k < kend && n < N) ? lb.at4(k, n) : make_float4(0.f, 0.f, 0.f, 0.f);
          rb[i][0] = x.x; rb[i][1] = x.y; rb[i][2] = x.z; rb[i][3] = x.w;
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) rb[i][j] = (k < kend && n + j < N) ? lb.at(k, n + j) : 0.f;
        }
      } else {                                  // 4 consecutive k of column n
        if constexpr (LB::kVec) {
          const float4 x = (n < N && k < kend) ? lb.at4(k, n) : make_float4(0.f, 0.f, 0.f, 0.f);
          rb[i][0] = x.x; rb[i][1] = x.y; rb[i][2] = x.z; rb[i][3] = x.w;
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) rb[i][j] = (n < N && k + j < kend) ? lb.at(k + j, n) : 0.f;
        }
      }
    }
  };
  auto store_b = [&](int buf) {
#pragma unroll
    for (int i = 0; i < VB; ++i) {
      int n, k;
      b_pos(tid + 256 * i, n, k);
      *reinterpret_cast<float4*>(Bs + b_off(buf, n, k)) = make_float4(rb[i][0], rb[i][1], rb[i][2], rb[i][3]);
    }
  };

  adhip_f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // Two LDS buffers: the panel prefetched into registers during the
  // products of the current panel is stored into the other buffer, so one
  // barrier per panel separates every write of a buffer from its last read.
  // One buffer (NBUF = 1): half the LDS, so a deeper panel still leaves
  // two blocks per compute unit; the next panel (already in registers) is
  // stored once every wave is done with the current one, a second barrier
  // per panel.
  const int lk = lane >> 5, lr = lane & 31;
  if (kbeg < kend) {
    load_a(kbeg);
    load_b(kbeg);
    store_a(0);
    store_b(0);
    __syncthreads();
    int cur = 0;
    for (int k0 = kbeg; k0 < kend; k0 += BK) {
      const bool more = k0 + BK < kend;
      if (more) {
        load_a(k0 + BK);
        load_b(k0 + BK);
      }
      // MFMA step s of the panel multiplies k = H * (lane / 32) + s: a lane
      // takes H consecutive k (any assignment of the panel's k to steps and
      // lane halves is a valid order of the sum, the same for A and B);
      // fragments are read 4 steps at a time.  The products run at raised
      // wave priority, so a wave in its product phase issues ahead of one
      // storing its panel (the two blocks of a compute unit alternate), and
      // iglp_opt(0) interleaves the fragment reads with the MFMAs (measured:
      // 4096^3 from 118.9 to 121.9 TFLOP/s)
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int q = 0; q < H / 4; ++q) {
        __builtin_amdgcn_iglp_opt(0);
        float af[TM][4], bf[TN][4];
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const int m = wm * (BM / 2) + i * 32 + lr;
          if constexpr (AR) {
            const float4 x = *reinterpret_cast<const float4*>(As + a_off(cur, m, H * lk + 4 * q));
            af[i][0] = x.x; af[i][1] = x.y; af[i][2] = x.z; af[i][3] = x.w;
          } else {
#pragma unroll
            for (int st = 0; st < 4; ++st) af[i][st] = As[a_off(cur, m, H * lk + 4 * q + st)];
          }
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int n = wn * (BN / 2) + j * 32 + lr;
          if constexpr (BR) {
            const float4 x = *reinterpret_cast<const float4*>(Bs + b_off(cur, n, H * lk + 4 * q));
            bf[j][0] = x.x; bf[j][1] = x.y; bf[j][2] = x.z; bf[j][3] = x.w;
          } else {
#pragma unroll
            for (int st = 0; st < 4; ++st) bf[j][st] = Bs[b_off(cur, n, H * lk + 4 * q + st)];
          }
        }
#pragma unroll
        for (int st = 0; st < 4; ++st)
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][st], bf[j][st], acc[i][j], 0, 0, 0);
      }
      __builtin_amdgcn_s_setprio(0);
      if constexpr (NBUF == 2) {
        if (more) {
          store_a(cur ^ 1);
          store_b(cur ^ 1);
        }
        __syncthreads();
        cur ^= 1;
      } else {
        if (more) {
          __syncthreads();
          store_a(0);
          store_b(0);
        }
        __syncthreads();
      }
    }
  }
  dp_epilogue<BM, BN>(epi, acc, smem, m0, n0, M, N, chunk);
}

// dp_quad<SPLIT, BK>: a DotProd for launches too small to fill the device (a
// few per-head products of 512 terms, one split weight gradient).  A 64x64
// tile per block leaves most compute units idle there, and each wave's chain
// of K/2 dependent MFMAs sets the launch's time.  Here a block of 4 waves
// takes a 32x32 output tile and splits each BK-deep K panel (128, or 64 for
// a short K) among its waves (wave w takes panel columns w*BK/4 onwards):
// four times the blocks, each wave's chain a quarter as long.  Panels are
// staged in one LDS buffer with the
// next panel prefetched into registers (two barriers per panel), laid out
// as in dp_mfma.  At the end the four 32x32 partial tiles go through LDS and
// each thread adds its 4 consecutive elements of one row in wave order, then
// runs the epilogue on them (float4 interface when EPI::kVec4, else per
// element).  SPLIT > 1 splits K into chunks over blockIdx.y as in dp_mfma.
constexpr int DPQ_RPITCH = 36;

template <int SPLIT, int BK, class LA, class LB, class EPI>
__device__ __forceinline__ void dp_quad(const LA& la, const LB& lb, const EPI& epi, int M, int N, int K) {
  static_assert(BK == 64 || BK == 128, "dp_quad panels are 64 or 128 deep");
  constexpr int BT = 32, KW = BK / 4, H = KW / 2;
  constexpr int V = BT * BK / 4 / 256;                // float4 loads per thread per operand
  constexpr bool AR = LA::kMode == 0, BR = LB::kMode == 1;
  constexpr int KP = BK + 4;
  constexpr int APITCH = AR ? KP : BT + 4, BPITCH = BR ? KP : BT + 4;
  constexpr int A_FLOATS = (AR ? BT : BK) * APITCH, B_FLOATS = (BR ? BT : BK) * BPITCH;
  constexpr int R_FLOATS = 4 * BT * DPQ_RPITCH;
  constexpr int S_FLOATS = A_FLOATS + B_FLOATS > R_FLOATS ? A_FLOATS + B_FLOATS : R_FLOATS;
  __shared__ __attribute__((aligned(16))) float smem[S_FLOATS];
  float* const As = smem;
  float* const Bs = smem + A_FLOATS;
  auto a_off = [](int m, int k) { return AR ? m * APITCH + k : k * APITCH + m; };
  auto b_off = [](int n, int k) { return BR ? n * BPITCH + k : k * BPITCH + n; };
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tiles_m = (M + BT - 1) / BT;
  int bx, by;
  dp_block_tile(bx, by);
  const int chunk = SPLIT > 1 ? by / tiles_m : 0;
  const int m0 = (SPLIT > 1 ? by % tiles_m : by) * BT, n0 = bx * BT;
  int kbeg = 0, kend = K;
  if constexpr (SPLIT > 1) {
    const int kc = ((K + SPLIT - 1) / SPLIT + BK - 1) / BK * BK;
    kbeg = chunk * kc;
    kend = kbeg + kc < K ? kbeg + kc : K;
  }
  float ra[V][4], rb[V][4];
  // float4 v of a panel: (row, k) of its first float
  auto a_pos = [](int v, int& m, int& k) {
    if constexpr (AR) { m = v / (BK / 4); k = 4 * (v % (BK / 4)); }
    else { k = v / (BT / 4); m = 4 * (v % (BT / 4)); }
  };
  auto b_pos = [](int v, int& n, int& k) {
    if constexpr (BR) { n = v / (BK / 4); k = 4 * (v % (BK / 4)); }
    else { k = v / (BT / 4); n = 4 * (v % (BT / 4)); }
  };
  auto load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < V; ++i) {
      int m, n, ka, kb;
      a_pos(tid + 256 * i, m, ka);
      b_pos(tid + 256 * i, n, kb);
      m += m0; ka += k0; n += n0; kb += k0;
      if constexpr (LA::kVec) {
        const float4 x = (m < M && ka < kend) ? la.at4(m, ka) : make_float4(0.f, 0.f, 0.f, 0.f);
        ra[i][0] = x.x; ra[i][1] = x.y; ra[i][2] = x.z; ra[i][3] = x.w;
      } else if constexpr (AR) {
#pragma unroll
        for (int j = 0; j < 4; ++j) ra[i][j] = (m < M && ka + j < kend) ? la.at(m, ka + j) : 0.f;
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) ra[i][j] = (ka < kend && m + j < M) ? la.at(m + j, ka) : 0.f;
      }
      if constexpr (LB::kVec) {
        const float4 x = (n < N && kb < kend) ? lb.at4(kb, n) : make_float4(0.f, 0.f, 0.f, 0.f);
        rb[i][0] = x.x; rb[i][1] = x.y; rb[i][2] = x.z; rb[i][3] = x.w;
      } else if constexpr (BR) {
#pragma unroll
        for (int j = 0; j < 4; ++j) rb[i][j] = (n < N && kb + j < kend) ? lb.at(kb + j, n) : 0.f;
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) rb[i][j] = (kb < kend && n + j < N) ? lb.at(kb, n + j) : 0.f;
      }
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int i = 0; i < V; ++i) {
      int m, n, ka, kb;
      a_pos(tid + 256 * i, m, ka);
      b_pos(tid + 256 * i, n, kb);
      *reinterpret_cast<float4*>(As + a_off(m, ka)) = make_float4(ra[i][0], ra[i][1], ra[i][2], ra[i][3]);
      *reinterpret_cast<float4*>(Bs + b_off(n, kb)) = make_float4(rb[i][0], rb[i][1], rb[i][2], rb[i][3]);
    }
  };

  adhip_f32x16 acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.f;
  const int lk = lane >> 5, lr = lane & 31;
  if (kbeg < kend) {
    load(kbeg);
    store();
    __syncthreads();
    for (int k0 = kbeg; k0 < kend; k0 += BK) {
      const bool more = k0 + BK < kend;
      if (more) load(k0 + BK);
      // MFMA step s of the wave's 32 panel columns multiplies column
      // KW * wave + H * (lane / 32) + s (the same assignment for A and B)
#pragma unroll
      for (int q = 0; q < H / 4; ++q) {
        float af[4], bf[4];
        const int kk = KW * wave + H * lk + 4 * q;
        if constexpr (AR) {
          const float4 x = *reinterpret_cast<const float4*>(As + a_off(lr, kk));
          af[0] = x.x; af[1] = x.y; af[2] = x.z; af[3] = x.w;
        } else {
#pragma unroll
          for (int st = 0; st < 4; ++st) af[st] = As[a_off(lr, kk + st)];
        }
        if constexpr (BR) {
          const float4 x = *reinterpret_cast<const float4*>(Bs + b_off(lr, kk));
          bf[0] = x.x; bf[1] = x.y; bf[2] = x.z; bf[3] = x.w;
        } else {
#pragma unroll
          for (int st = 0; st < 4; ++st) bf[st] = Bs[b_off(lr, kk + st)];
        }
#pragma unroll
        for (int st = 0; st < 4; ++st) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(af[st], bf[st], acc, 0, 0, 0);
      }
      if (more) {
        __syncthreads();
        store();
      }
      __syncthreads();
    }
  }
  // the four waves' partial tiles: lane holds column lane % 32 and rows
  // 8*(r/4) + 4*(lane/32) + r%4 of its wave's tile
  __syncthreads();
  float* const red = smem;
#pragma unroll
  for (int r = 0; r < 16; ++r)
    red[(wave * BT + 8 * (r >> 2) + 4 * lk + (r & 3)) * DPQ_RPITCH + lr] = acc[r];
  __syncthreads();
  const int row = tid >> 3, c4 = 4 * (tid & 7);
  float4 v = *reinterpret_cast<const float4*>(red + row * DPQ_RPITCH + c4);
#pragma unroll
  for (int w = 1; w < 4; ++w) {
    const float4 x = *reinterpret_cast<const float4*>(red + (w * BT + row) * DPQ_RPITCH + c4);
    v.x = v.x + x.x; v.y = v.y + x.y; v.z = v.z + x.z; v.w = v.w + x.w;
  }
  const int gm = m0 + row, gn = n0 + c4;
  if (gm >= M) return;
  constexpr int NL = EPI::kLoads > 0 ? EPI::kLoads : 1;
  if constexpr (EPI::kVec4) {
    if (gn < N) {
      float4 lv[NL];
      epi.load4(gm, gn, lv);
      epi.vec(v, gm, gn, chunk, lv);
    }
  } else {
    const float vs[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (gn + j < N) {
        float lv[NL];
        epi.load(gm, gn + j, lv);
        epi(vs[j], gm, gn + j, chunk, lv);
      }
  }
}

// dp_skinny<MR>: a DotProd with at most MR rows (a product like [2,255] x
// [255,255], where an MFMA tile would idle on the short side and its K
// panels and barriers would set the time).  A block of 256 lanes takes 16
// columns; the 16 lanes of a column split K (lane s takes k = s, s + 16,
// ...), so for K <= 256 a lane has every load in flight at once; the 16
// partial sums of each row combine by butterfly within the group, and lane
// s < M of the group runs the epilogue of row s (scalar EPI interface).
template <int MR, class LA, class LB, class EPI>
__device__ __forceinline__ void dp_skinny(const LA& la, const LB& lb, const EPI& epi, int M, int N, int K) {
  const int t = threadIdx.x;
  const int s = t & 15;
  const int n = blockIdx.x * 16 + (t >> 4);
  float acc[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) acc[m] = 0.f;
  if (n < N) {
#pragma unroll 4
    for (int k = s; k < K; k += 16) {
      const float b = lb.at(k, n);
#pragma unroll
      for (int m = 0; m < MR; ++m)
        if (m < M) acc[m] = acc[m] + la.at(m, k) * b;
    }
  }
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) acc[m] = acc[m] + __shfl_xor(acc[m], off, 16);
  if (n < N && s < M) {
    float v = acc[0];
#pragma unroll
    for (int m = 1; m < MR; ++m)
      if (m == s) v = acc[m];
    constexpr int NL = EPI::kLoads > 0 ? EPI::kLoads : 1;
    float lv[NL];
    epi.load(s, n, lv);
    epi(v, s, n, 0, lv);
  }
}

// dp_direct: a DotProd with a short K (at most a few terms, such as the
// [255,2] x [2,255] weight gradients of a batch of 2): one lane per output,
// the K products summed in order, then the scalar epilogue; no tile, no LDS.
template <class LA, class LB, class EPI>
__device__ __forceinline__ void dp_direct(const LA& la, const LB& lb, const EPI& epi, int M, int N, int K) {
  const unsigned long long g = (unsigned long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= (unsigned long long)M * (unsigned long long)N) return;
  const int m = (int)(g / (unsigned long long)N), n = (int)(g % (unsigned long long)N);
  float acc = 0.f;
  for (int k = 0; k < K; ++k) acc = acc + la.at(m, k) * lb.at(k, n);
  constexpr int NL = EPI::kLoads > 0 ? EPI::kLoads : 1;
  float lv[NL];
  epi.load(m, n, lv);
  epi(acc, m, n, 0, lv);
}

// ---------------------------------------------------------------- bf16 DotProd
// An option, not the reference: operands rounded to bfloat16 (nearest even),
// products accumulated in fp32 by v_mfma_f32_32x32x16_bf16.
typedef __bf16 adhip_bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ unsigned adhip_pack2_bf16(float a, float b) {
  return (unsigned)__builtin_bit_cast(unsigned short, (__bf16)a) |
         ((unsigned)__builtin_bit_cast(unsigned short, (__bf16)b) << 16);
}

// pack_bf16<ROLE>: a DotProd operand as a k-contiguous bf16 matrix
// dst[r * KPAD + k] for r < 64 * gridDim.y, k < 64 * gridDim.x (KPAD), zero
// outside R x K.  ROLE 0: A, LD::at(r, k); ROLE 1: B, LD::at(k, r).  Each
// block moves a 64 x 64 tile through LDS: loads coalesced along the
// operand's contiguous axis, stores of 16 consecutive k per lane.
template <int ROLE, class LD>
__device__ __forceinline__ void pack_bf16(const LD& ld, __bf16* __restrict__ dst, int R, int K, int KPAD) {
  __shared__ float tile[64][65];
  constexpr bool rows_contig = ROLE == 0 ? LD::kMode == 1 : LD::kMode == 0;
  const int t = threadIdx.x;
  const int r0 = blockIdx.y * 64, k0 = blockIdx.x * 64;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    int rl, kl;
    if constexpr (rows_contig) { rl = t & 63; kl = (t >> 6) + 4 * i; }
    else { kl = t & 63; rl = (t >> 6) + 4 * i; }
    const int r = r0 + rl, k = k0 + kl;
    float v = 0.f;
    if (r < R && k < K) {
      if constexpr (ROLE == 0) v = ld.at(r, k);
      else v = ld.at(k, r);
    }
    tile[rl][kl] = v;
  }
  __syncthreads();
  const int rl = t >> 2, kq = (t & 3) * 16;
  uint4 w[2];
  unsigned* u = reinterpret_cast<unsigned*>(w);
#pragma unroll
  for (int j = 0; j < 8; ++j) u[j] = adhip_pack2_bf16(tile[rl][kq + 2 * j], tile[rl][kq + 2 * j + 1]);
  uint4* d = reinterpret_cast<uint4*>(dst + (size_t)(r0 + rl) * KPAD + k0 + kq);
  d[0] = w[0];
  d[1] = w[1];
}

// dp_bf16<BM, BN, SPLIT, BK>: C[m][n] = sum_k A[m][k] * B[n][k] over packed
// operands (rows padded to the tile, KPAD bf16 per row, zero padded).  K
// panels of BK in two LDS buffers ([row][k], pitch BK + 8 bf16); per panel,
// BK/16 MFMA steps of 16 k, a lane taking 8 consecutive k (one 16-byte read)
// per 32-row tile.  Tile order, K split and epilogue as dp_mfma.
template <int BM, int BN, int SPLIT, int BK, class EPI>
__device__ __forceinline__ void dp_bf16(const __bf16* __restrict__ A, const __bf16* __restrict__ B, int KPAD,
                                        const EPI& epi, int M, int N) {
  static_assert(BK % 32 == 0, "K panel must be a multiple of 32");
  constexpr int TM = BM / 64, TN = BN / 64, KP = BK + 8, CH = BK / 8;
  constexpr int VA = BM * BK / 8 / 256, VB = BN * BK / 8 / 256;   // 16-byte loads per thread
  static_assert(VA >= 1 && VB >= 1, "tile too small for 256 threads");
  constexpr int A_HALVES = 2 * BM * KP, B_HALVES = 2 * BN * KP;
  constexpr int C_FLOATS = EPI::kVec4 ? 4 * 32 * DP_CPITCH : 0;
  constexpr int S_FLOATS = (A_HALVES + B_HALVES) / 2 > C_FLOATS ? (A_HALVES + B_HALVES) / 2 : C_FLOATS;
  __shared__ __attribute__((aligned(16))) float smem[S_FLOATS];
  __bf16* const As = reinterpret_cast<__bf16*>(smem);
  __bf16* const Bs = As + A_HALVES;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int lk = lane >> 5, lr = lane & 31;
  const int tiles_m = (M + BM - 1) / BM;
  int bx, by;
  dp_block_tile(bx, by);
  const int chunk = SPLIT > 1 ? by / tiles_m : 0;
  const int m0 = (SPLIT > 1 ? by % tiles_m : by) * BM, n0 = bx * BN;
  int kbeg = 0, kend = KPAD;
  if constexpr (SPLIT > 1) {
    const int kc = ((KPAD + SPLIT - 1) / SPLIT + BK - 1) / BK * BK;
    kbeg = chunk * kc;
    kend = kbeg + kc < KPAD ? kbeg + kc : KPAD;
  }
  uint4 ra[VA], rb[VB];
  auto load = [&](int k0) {
#pragma unroll
    for (int i = 0; i < VA; ++i) {
      const int v = tid + 256 * i;
      ra[i] = *reinterpret_cast<const uint4*>(A + (size_t)(m0 + v / CH) * KPAD + k0 + 8 * (v % CH));
    }
#pragma unroll
    for (int i = 0; i < VB; ++i) {
      const int v = tid + 256 * i;
      rb[i] = *reinterpret_cast<const uint4*>(B + (size_t)(n0 + v / CH) * KPAD + k0 + 8 * (v % CH));
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < VA; ++i) {
      const int v = tid + 256 * i;
      *reinterpret_cast<uint4*>(As + (buf * BM + v / CH) * KP + 8 * (v % CH)) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < VB; ++i) {
      const int v = tid + 256 * i;
      *reinterpret_cast<uint4*>(Bs + (buf * BN + v / CH) * KP + 8 * (v % CH)) = rb[i];
    }
  };
  adhip_f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  if (kbeg < kend) {
    load(kbeg);
    store(0);
    __syncthreads();
    int cur = 0;
    for (int k0 = kbeg; k0 < kend; k0 += BK) {
      const bool more = k0 + BK < kend;
      if (more) load(k0 + BK);
      __builtin_amdgcn_s_setprio(1);          // as in dp_mfma
#pragma unroll
      for (int st = 0; st < BK / 16; ++st) {
        __builtin_amdgcn_iglp_opt(0);
        adhip_bf16x8 af[TM], bf[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
          af[i] = *reinterpret_cast<const adhip_bf16x8*>(As + (cur * BM + wm * (BM / 2) + i * 32 + lr) * KP + 16 * st + 8 * lk);
#pragma unroll
        for (int j = 0; j < TN; ++j)
          bf[j] = *reinterpret_cast<const adhip_bf16x8*>(Bs + (cur * BN + wn * (BN / 2) + j * 32 + lr) * KP + 16 * st + 8 * lk);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
      }
      __builtin_amdgcn_s_setprio(0);
      if (more) store(cur ^ 1);
      __syncthreads();
      cur ^= 1;
    }
  }
  dp_epilogue<BM, BN>(epi, acc, smem, m0, n0, M, N, chunk);
}

// ---------------------------------------------------------------- Reduce+Elw
// LD::at(x, y) loads element y of reduced row x; LD::at4 four consecutive y.
// LD::inc(y) is false for elements the reference's work-group tree drops.
//
// reduce_rows: waves stride over the rows (a bounded grid keeps every wave
// busy across several rows); per row, each lane keeps up to sixteen float4
// loads in flight, then a butterfly over the wave; lane 0 runs the epilogue.
template <int OP, class LD, class EPI>
__device__ __forceinline__ void reduce_rows(const LD& ld, const EPI& epi, unsigned V, unsigned R,
                                            bool pad_zero) {
  const unsigned lane = threadIdx.x & 63;
  const unsigned waves = gridDim.x * (blockDim.x >> 6);
  const float id = OP == 0 ? 0.f : -__builtin_huge_valf();
  for (unsigned row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); row < V; row += waves) {
    float acc = id;
    if constexpr (LD::kVec) {
      float a[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) a[u] = id;
      // 16 float4 loads in flight per lane; the last round is predicated
      // (identity for the loads past the row)
      const float4 idv = make_float4(id, id, id, id);
      for (unsigned y0 = lane * 4; y0 < R; y0 += 16 * 256) {
        float4 v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = y0 + u * 256 < R ? ld.at4(row, y0 + u * 256) : idv;
#pragma unroll
        for (int u = 0; u < 16; ++u)
          a[u & 7] = rop<OP>(rop<OP>(rop<OP>(rop<OP>(a[u & 7], v[u].x), v[u].y), v[u].z), v[u].w);
      }
      acc = rop<OP>(rop<OP>(rop<OP>(a[0], a[1]), rop<OP>(a[2], a[3])),
                    rop<OP>(rop<OP>(a[4], a[5]), rop<OP>(a[6], a[7])));
    } else {
      for (unsigned y = lane; y < R; y += 64)
        if (ld.inc(y)) acc = rop<OP>(acc, ld.at(row, y));
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) acc = rop<OP>(acc, __shfl_xor(acc, off, 64));
    if (OP == 1 && pad_zero) acc = fmaxf(acc, 0.f);
    if (lane == 0) epi(acc, row, 0);
  }
}

// reduce_cols: a block covers 64 columns and G row groups: with LD::kVecX
// 16 lanes per group load 4 consecutive columns each as one float4
// (G = 16), else 64 lanes load one column each (G = 4); group g takes rows
// g, g+G, ..., a lane keeps 8 rows' loads in flight, and the groups combine
// through LDS in order.  SPLIT > 1 splits the rows into SPLIT chunks
// (blockIdx.y) whose results go to the epilogue with the chunk index and
// without the zero padding of MAX (applied once the chunks are combined).
template <int OP, int SPLIT, class LD, class EPI>
__device__ __forceinline__ void reduce_cols(const LD& ld, const EPI& epi, unsigned V, unsigned R,
                                            bool pad_zero) {
  constexpr int W = LD::kVecX ? 4 : 1;         // columns per lane
  constexpr int L = 64 / W;                    // lanes per row group
  constexpr int G = 256 / L;                   // row groups per block
  __shared__ float part[G][64];
  const unsigned t = threadIdx.x;
  const unsigned grp = t / L, sub = t % L;
  const unsigned col0 = blockIdx.x * 64 + sub * W;
  unsigned ybeg = 0, yend = R;
  if constexpr (SPLIT > 1) {
    const unsigned rc = (R + SPLIT - 1) / SPLIT;
    ybeg = blockIdx.y * rc;
    yend = ybeg + rc < R ? ybeg + rc : R;
  }
  const float id = OP == 0 ? 0.f : -__builtin_huge_valf();
  float acc[W];
#pragma unroll
  for (int w = 0; w < W; ++w) acc[w] = id;
  if constexpr (W == 4) {
    // V % 4 == 0: a lane's 4 columns are all in range or all out
    if (col0 < V) {
      unsigned y = ybeg + grp;
      for (; y + 7 * G < yend; y += 8 * G) {
        float4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = ld.at4(col0, y + G * u);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          acc[0] = rop<OP>(acc[0], v[u].x);
          acc[1] = rop<OP>(acc[1], v[u].y);
          acc[2] = rop<OP>(acc[2], v[u].z);
          acc[3] = rop<OP>(acc[3], v[u].w);
        }
      }
      for (; y < yend; y += G) {
        const float4 v = ld.at4(col0, y);
        acc[0] = rop<OP>(acc[0], v.x);
        acc[1] = rop<OP>(acc[1], v.y);
        acc[2] = rop<OP>(acc[2], v.z);
        acc[3] = rop<OP>(acc[3], v.w);
      }
    }
  } else {
    if (col0 < V)
      for (unsigned y = ybeg + grp; y < yend; y += G)
        if (ld.inc(y)) acc[0] = rop<OP>(acc[0], ld.at(col0, y));
  }
#pragma unroll
  for (int w = 0; w < W; ++w) part[grp][sub * W + w] = acc[w];
  __syncthreads();
  if (t < 64) {
    const unsigned col = blockIdx.x * 64 + t;
    if (col < V) {
      float a = part[0][t];
#pragma unroll
      for (int g = 1; g < G; ++g) a = rop<OP>(a, part[g][t]);
      if (SPLIT == 1 && OP == 1 && pad_zero) a = fmaxf(a, 0.f);
      epi(a, col, (int)blockIdx.y);
    }
  }
}

}  // namespace adhip
