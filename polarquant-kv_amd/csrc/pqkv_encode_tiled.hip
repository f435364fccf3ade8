// Register-blocked exact encoder: the FMA-chain rotation of the reference's
// encode kernel (csrc/flash_turboquant.cu:132-137, rot[j] = fp32 FMA chain
// over k = 0..d-1 of x[k] * R[j][k]) computed as a tiled product, then the
// quantiser of csrc/flash_turboquant.cu:141-170 on the values in registers.
//
// Work split. A workgroup of 8 waves takes VS vectors per step (128 at
// d = 128, 256 at d = 64; a half or a quarter of that when full-size steps
// would leave compute units without one). Lane row tv = tid / 16 owns VT
// consecutive vectors of the step (4 / 8, 2 / 4 or 1 / 2) and lane tj = tid % 16 of the row owns output
// coordinates j = 64 g + 4 tj + i (g < d / 64, i < 4): 32 accumulators per
// thread, each the chain of one (vector, coordinate) over k ascending, so
// every rotated value is bit-identical to the one-chain form. Per k a thread
// reads its VT input values (one 16-byte LDS read per vector per four k) and
// its 4 d / 64 values of row k of R^T (16-byte reads; the 16 lanes of a row
// read 256 contiguous bytes), three LDS reads per 32 FMAs at d = 128 where
// the one-vector-per-thread form needs one per four.
//
// LDS: R^T for the launch (64 KB at d = 128), the input in 32-coordinate
// chunks (double-buffered, loaded through registers one chunk ahead, one
// barrier per chunk), the switch-point cell table and the step's output.
// One workgroup per compute unit (2 waves per SIMD).
//
// Quantiser, per vector, on its 16 lanes:
//   - radius: the reference's 128-slot tree of squares. The step s = 64
//     pairs coordinates j and j + 64 of one thread; the steps s = 32 .. 4
//     pair lanes tj and tj +- s / 4, done as DPP row rotations by 8, 4, 2, 1
//     (after the step by s the lanes' partial sums repeat with period s / 4,
//     so a rotation pairs each lane with a holder of slot t ^ s; IEEE
//     addition commutes); s = 2, 1 pair the thread's own four slots. Then
//     the correctly rounded sqrt (fp64 root rounded once);
//   - index: the switch-point cell table of pqkv_cells.h with the Markstein
//     direction (or a per-coordinate division for radii outside its range),
//     the reference's scan when the table refuses the codebook.
// Output: block_pq4 / block_pq2 vectors (fp16 radius per block) or the
// reference's SoA codes (packed[p] = code(2p) | code(2p+1) << 4) with fp32
// radii, staged in LDS and stored one step later, 16-byte pieces for one
// aligned run of vectors, dwords otherwise. QJL keys add the sign sketch of
// the residual (src/polarquant_kv_cuda/compress_kernel.py:166-175) as a
// second tiled product (encode_tiled_kernel's QJL flag).
#include <type_traits>

#include "pqkv_cells.h"
#include "pqkv_device.h"
#include "pqkv_launch.h"

namespace pqkv {

namespace {

constexpr int kTW = 8;              // waves per workgroup
constexpr int kTT = kTW * 64;       // threads per workgroup
constexpr int kTK = 32;             // input coordinates per staged chunk
constexpr int kTXP = kTK + 4;       // floats per staged vector chunk (padded: 16-byte aligned rows in
                                    // different banks)

// SH: the vectors per thread and step halved SH times (0..2), for launches
// with fewer full-size steps than compute units.
template <int D, int SH>
struct TiledShape {
  static constexpr int NG = D / 64;               // 64-coordinate groups per thread
  static constexpr int VT = (8 / NG) >> SH;       // vectors per thread
  static constexpr int VS = 32 * VT;              // vectors per step (32 rows of 16 lanes)
  static constexpr int NC = D / kTK;              // chunks per step
};

// Lane l of a 16-lane row receives lane (l + N) % 16's value (DPP row_ror).
template <int N>
__device__ __forceinline__ float row_ror(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x120 + N, 0xF, 0xF, true));
}

typedef __attribute__((address_space(3))) uint8_t lds_u8;
typedef __attribute__((address_space(3))) uint32_t lds_u32;

}  // namespace

// OUT: 4 / 2 = block_pq4 / block_pq2 vectors through a's output addressing;
// 0 = SoA codes at a.blocks (d / 2 bytes per vector) and fp32 radii at
// soa_radius, one run of n_inner vectors. nl levels (<= 16).
// QJL (keys, m = d projections, half-size steps): after a step's quantiser
// each thread writes its residuals e = y - r c[code] (fp32 r) to LDS, and
// the projections P_rot e run as a second tiled product over k ascending,
// P_rot staged in 16-coordinate chunks (transposed, double-buffered); sign
// bit m = (P_rot e)[m] >= 0, LSB first, stored one step later like the
// blocks.
template <int D, int OUT, typename TIN, int SH, bool QJL = false>
__global__ void __launch_bounds__(kTT, 1) encode_tiled_kernel(const EncodeArgs a, const int nl, float *soa_radius) {
  using S = TiledShape<D, SH>;
  constexpr int NG = S::NG, VT = S::VT, VS = S::VS, NC = S::NC;
  constexpr int VB = OUT == 0 ? D / 2 : vector_bytes(D, OUT);   // output bytes per vector
  constexpr int BB = OUT == 0 ? 0 : block_bytes(OUT);
  constexpr int PPV = kTK * (int)sizeof(TIN) / 16;               // 16-byte input pieces per vector chunk
  constexpr int EPP = 16 / (int)sizeof(TIN);                     // input elements per piece
  constexpr int NPC = VS * PPV;                                  // input pieces per chunk
  constexpr int NP = (NPC + kTT - 1) / kTT;                      // pieces per thread per chunk
  static_assert(NPC % kTT == 0 || NP == 1, "threads past the chunk's pieces take none");
  static_assert(NC % 2 == 0, "chunk c of every step in buffer c % 2");
  constexpr int SB = D / 8;          // sign bytes per vector
  constexpr int PK = 16;             // projection k per staged chunk of P_rot
  constexpr int NPK = D / PK;        // chunks per projection
  constexpr int ESP = D + 4;         // floats per residual row (padded like xs)
  static_assert(VT >= 1, "at least one vector per thread");
  static_assert(!QJL || (SH >= 1 && OUT != 0), "QJL keys: blocks, half-size or smaller steps");
  static_assert(PK * D / 4 <= kTT, "one P_rot piece per thread and chunk");
  __shared__ __attribute__((aligned(16))) float rt[D * D];           // rt[k * D + j] = R[j][k]
  __shared__ __attribute__((aligned(16))) float xs[2][VS * kTXP];    // xs[b][v * kTXP + kk]
  __shared__ __attribute__((aligned(16))) uint8_t stage[VS * VB];
  __shared__ uint2 cells[kECellSlots];
  __shared__ float cb[16], thr[16];
  __shared__ int ucell[16];
  __shared__ int table_ok;
  __shared__ __attribute__((aligned(16))) float es[QJL ? VS * ESP : 4];        // residuals e[v][k]
  __shared__ __attribute__((aligned(16))) float pt[2][QJL ? PK * D : 4];       // pt[b][kk * D + m] = P_rot[m][PK pc + kk]
  __shared__ __attribute__((aligned(16))) uint8_t sstage[QJL ? VS * SB : 16];  // the step's sign bytes

  const int tid = threadIdx.x;
  const int tj = tid & 15, tv = tid >> 4;
  const uint32_t n = (uint32_t)(a.n_outer * a.n_inner);
  const uint32_t steps = (n + VS - 1) / VS;
  const FastDiv by_inner((uint32_t)a.n_inner);
  const TIN *x = (const TIN *)a.x;
  bool use_table = false;   // whether the switch-point table holds (set after its build)

  // ---- input: piece p of this thread is piece q % PPV of vector q / PPV of
  // the step, q = tid + kTT p ----
  const TIN *src[NP];
  auto set_rows = [&](uint32_t s) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int q = tid + kTT * p;
      const uint32_t v = s * VS + q / PPV;
      if (q < NPC && v < n) {
        const uint32_t vo = by_inner.div(v), vi = v - vo * (uint32_t)a.n_inner;
        src[p] = x + (int64_t)vo * a.x_outer_stride + (int64_t)vi * D + EPP * (q % PPV);
      } else {
        src[p] = nullptr;
      }
    }
  };
  u32x4 pre[NP];
  auto load = [&](int c) {
#pragma unroll
    for (int p = 0; p < NP; ++p) pre[p] = src[p] ? *(const u32x4 *)(src[p] + c * kTK) : u32x4{0, 0, 0, 0};
  };
  auto store_x = [&](int b) {
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int q = tid + kTT * p;
      if (q >= NPC) continue;
      float *dst = &xs[b][(q / PPV) * kTXP + EPP * (q % PPV)];
      if constexpr (sizeof(TIN) == 4) {
        *(float4_t *)dst = __builtin_bit_cast(float4_t, pre[p]);
      } else if constexpr (__is_same(TIN, bf16_t)) {
        const u32x4 w = pre[p];
        *(float4_t *)dst = float4_t{bf16_to_float(w[0] & 0xFFFFu), bf16_to_float(w[0] >> 16),
                                    bf16_to_float(w[1] & 0xFFFFu), bf16_to_float(w[1] >> 16)};
        *(float4_t *)(dst + 4) = float4_t{bf16_to_float(w[2] & 0xFFFFu), bf16_to_float(w[2] >> 16),
                                          bf16_to_float(w[3] & 0xFFFFu), bf16_to_float(w[3] >> 16)};
      } else {
        const half8_t h = __builtin_bit_cast(half8_t, pre[p]);
        *(float4_t *)dst = float4_t{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
        *(float4_t *)(dst + 4) = float4_t{(float)h[4], (float)h[5], (float)h[6], (float)h[7]};
      }
    }
  };

  // ---- the tiled FMA chains: acc[u][g][i] for vector VT tv + u, coordinate
  // 64 g + 4 tj + i ----
  float acc[VT][NG][4];
  auto compute = [&](int b, int c) {
    const float *xb = &xs[b][(VT * tv) * kTXP];
    const float *rb = &rt[(c * kTK) * D + 4 * tj];
    // operands of four k: VT input 4-vectors and 4 NG R^T 4-vectors, the
    // next four's read while these feed the FMAs
    float4_t xv[VT], rv[4][NG];
    auto read = [&](int k4, float4_t (&xo)[VT], float4_t (&ro)[4][NG]) {
#pragma unroll
      for (int u = 0; u < VT; ++u) xo[u] = *(const float4_t *)(xb + u * kTXP + 4 * k4);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int g = 0; g < NG; ++g) ro[kk][g] = *(const float4_t *)(rb + (4 * k4 + kk) * D + 64 * g);
    };
    read(0, xv, rv);
#pragma nounroll
    for (int k4 = 0; k4 < kTK / 4; ++k4) {
      float4_t xn[VT], rn[4][NG];
      if (k4 + 1 < kTK / 4) read(k4 + 1, xn, rn);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int u = 0; u < VT; ++u)
#pragma unroll
          for (int g = 0; g < NG; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[u][g][i] = __builtin_fmaf(xv[u][kk], rv[kk][g][i], acc[u][g][i]);
#pragma unroll
      for (int u = 0; u < VT; ++u) xv[u] = xn[u];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int g = 0; g < NG; ++g) rv[kk][g] = rn[kk][g];
    }
  };

  // ---- quantiser: step s's vectors from acc into stage ----
  auto quantise = [&](uint32_t s) {
#pragma clang fp contract(off)
#pragma unroll
    for (int u = 0; u < VT; ++u) {
      const int vl = VT * tv + u;
      float sq[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p0 = acc[u][0][i] * acc[u][0][i];
        if constexpr (NG == 2) {
          const float p1 = acc[u][1][i] * acc[u][1][i];
          sq[i] = p0 + p1;   // tree step s = 64
        } else {
          sq[i] = p0;
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) sq[i] = sq[i] + row_ror<8>(sq[i]);   // s = 32
#pragma unroll
      for (int i = 0; i < 4; ++i) sq[i] = sq[i] + row_ror<4>(sq[i]);   // s = 16
#pragma unroll
      for (int i = 0; i < 4; ++i) sq[i] = sq[i] + row_ror<2>(sq[i]);   // s = 8
#pragma unroll
      for (int i = 0; i < 4; ++i) sq[i] = sq[i] + row_ror<1>(sq[i]);   // s = 4
      const float s2a = sq[0] + sq[2], s2b = sq[1] + sq[3];           // s = 2
      const float tot = s2a + s2b;                                    // s = 1
      const float r = (float)__builtin_sqrt((double)tot);
      int code[NG][4];
      if (use_table) {
        if (markstein_radius(r)) {
          const float inv = r > 1e-30f ? __fdiv_rn(1.0f, r) : 0.0f;
#pragma unroll
          for (int g = 0; g < NG; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i) code[g][i] = table_code(cells, dir_markstein(acc[u][g][i], r, inv));
        } else {
#pragma unroll
          for (int g = 0; g < NG; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i) code[g][i] = table_code(cells, dir_divided(acc[u][g][i], r));
        }
      } else {
        const bool nz = r > 1e-30f;
#pragma unroll
        for (int g = 0; g < NG; ++g)
#pragma unroll
          for (int i = 0; i < 4; ++i) code[g][i] = scan_index_rolled(nz ? __fdiv_rn(acc[u][g][i], r) : 0.0f, cb, nl);
      }
      lds_u8 *sv = (lds_u8 *)stage + vl * VB;
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        if constexpr (OUT == 0) {
          *(__attribute__((address_space(3))) uint16_t *)(sv + 32 * g + 2 * tj) =
              (uint16_t)(code[g][0] | (code[g][1] << 4) | (code[g][2] << 8) | (code[g][3] << 12));
        } else {
          const int blk = 2 * g + (tj >> 3);
          lds_u8 *bp = sv + blk * BB;
          if constexpr (OUT == 4)
            *(__attribute__((address_space(3))) uint16_t *)(bp + 2 + 2 * (tj & 7)) =
                (uint16_t)(code[g][0] | (code[g][1] << 4) | (code[g][2] << 8) | (code[g][3] << 12));
          else
            bp[2 + (tj & 7)] = (uint8_t)(code[g][0] | (code[g][1] << 2) | (code[g][2] << 4) | (code[g][3] << 6));
          if ((tj & 7) == 0) *(__attribute__((address_space(3))) uint16_t *)bp = radius_half_bits(r);
        }
      }
      if constexpr (OUT == 0) {
        const uint32_t v = s * VS + vl;
        if (tj == 0 && v < n) soa_radius[v] = r;
      }
      if constexpr (QJL) {
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          float4_t e;
#pragma unroll
          for (int i = 0; i < 4; ++i) e[i] = __builtin_fmaf(-r, cb[code[g][i]], acc[u][g][i]);
          *(float4_t *)&es[vl * ESP + 64 * g + 4 * tj] = e;
        }
      }
    }
  };

  // ---- QJL: P_rot chunk pc (coordinates PK pc ..) through registers into
  // pt[b]; thread t < PK D / 4 takes row m = t % D, 4 coordinates ----
  float4_t ppre;
  auto load_p = [&](int pc) {
    if (tid < PK * D / 4) ppre = *(const float4_t *)(a.p_rot + (int64_t)(tid % D) * D + PK * pc + 4 * (tid / D));
  };
  auto store_p = [&](int b) {
    if (tid < PK * D / 4) {
#pragma unroll
      for (int e = 0; e < 4; ++e) pt[b][(4 * (tid / D) + e) * D + tid % D] = ppre[e];
    }
  };
  // projections acc2[u][g][i] of vector VT tv + u, m = 64 g + 4 tj + i: the
  // FMA chain over k ascending, k = PK pc .. PK pc + PK - 1 in this call
  float acc2[VT][NG][4];
  auto project = [&](int b, int pc) {
    const float *eb = &es[(VT * tv) * ESP + PK * pc];
    const float *pb = &pt[b][4 * tj];
    float4_t ev[VT], pv[4][NG];
    auto read = [&](int k4, float4_t (&eo)[VT], float4_t (&po)[4][NG]) {
#pragma unroll
      for (int u = 0; u < VT; ++u) eo[u] = *(const float4_t *)(eb + u * ESP + 4 * k4);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int g = 0; g < NG; ++g) po[kk][g] = *(const float4_t *)(pb + (4 * k4 + kk) * D + 64 * g);
    };
    read(0, ev, pv);
#pragma nounroll
    for (int k4 = 0; k4 < PK / 4; ++k4) {
      float4_t en[VT], pn[4][NG];
      if (k4 + 1 < PK / 4) read(k4 + 1, en, pn);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int u = 0; u < VT; ++u)
#pragma unroll
          for (int g = 0; g < NG; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc2[u][g][i] = __builtin_fmaf(ev[u][kk], pv[kk][g][i], acc2[u][g][i]);
#pragma unroll
      for (int u = 0; u < VT; ++u) ev[u] = en[u];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int g = 0; g < NG; ++g) pv[kk][g] = pn[kk][g];
    }
  };
  // sign bytes of step s into sstage: lane tj holds bits 4 (tj & 1) .. + 3
  // of byte 8 g + tj / 2; the even lane of each pair writes the byte
  auto signs = [&] {
#pragma unroll
    for (int u = 0; u < VT; ++u)
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        uint32_t nib = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) nib |= (acc2[u][g][i] >= 0.0f ? 1u : 0u) << i;
        const uint32_t other = (uint32_t)__builtin_amdgcn_mov_dpp((int)nib, 0xB1, 0xF, 0xF, true);  // quad_perm [1,0,3,2]
        if ((tj & 1) == 0) sstage[(VT * tv + u) * SB + 8 * g + (tj >> 1)] = (uint8_t)(nib | (other << 4));
      }
  };

  // ---- step s's output from a stage (W bytes per vector) to memory: one
  // run of 16-byte pieces when the outputs are one aligned run, else dwords
  // through the output addressing ----
  auto flush_any = [&](auto wc, uint32_t s, const lds_u8 *stg, uint8_t *outb, uint8_t *const *pages, int64_t stride,
                       bool r16) {
    constexpr int W = decltype(wc)::value;
    const uint32_t v0 = s * VS;
    const int nv = (int)min(n - v0, (uint32_t)VS);
    if (r16) {
      const int nbytes = nv * W;
      uint8_t *base = outb + (int64_t)v0 * W;
#pragma unroll
      for (int it = 0; it < (VS * W / 16 + kTT - 1) / kTT; ++it) {
        const int p = tid + kTT * it;
        if (16 * p + 16 <= nbytes) {
          *(u32x4 *)(base + 16 * p) = *(const __attribute__((address_space(3))) u32x4 *)(stg + 16 * p);
        } else if (16 * p < nbytes) {
          for (int c = 0; c < 4 && 16 * p + 4 * c < nbytes; ++c)
            *(uint32_t *)(base + 16 * p + 4 * c) = *(const lds_u32 *)(stg + 16 * p + 4 * c);
        }
      }
      return;
    }
    constexpr int DW = W / 4;
#pragma unroll
    for (int it = 0; it < (VS * DW + kTT - 1) / kTT; ++it) {
      const int q = tid + kTT * it;
      const int vl = q / DW, c = q - vl * DW;
      if (q < VS * DW && vl < nv) {
        const uint32_t v = v0 + vl;
        const uint32_t vo = by_inner.div(v), vi = v - vo * (uint32_t)a.n_inner;
        *(uint32_t *)(encode_out_addr(a, outb, pages, stride, vo, vi, W) + 4 * c) = *(const lds_u32 *)(stg + vl * W + 4 * c);
      }
    }
  };
  const bool run16 = a.n_outer <= 1 && a.pages == nullptr && ((uintptr_t)a.blocks & 15) == 0;
  const bool srun16 = QJL && a.n_outer <= 1 && a.qjl_pages == nullptr && ((uintptr_t)a.qjl & 15) == 0;
  auto flush = [&](uint32_t s) {
    flush_any(std::integral_constant<int, VB>{}, s, (const lds_u8 *)stage, a.blocks, a.pages, a.blocks_outer_stride,
              run16);
  };
  auto flush_signs = [&](uint32_t s) {
    if constexpr (QJL)
      flush_any(std::integral_constant<int, SB>{}, s, (const lds_u8 *)sstage, a.qjl, a.qjl_pages, a.qjl_outer_stride,
                srun16);
  };

  // ---- pipeline: chunk c of step s computes from xs[c % 2] while chunk
  // c + 1 (or the next step's chunk 0) is in flight into registers; one
  // barrier per chunk. The host launches at most `steps` workgroups. ----
  uint32_t s = blockIdx.x;
  const float cbv = tid < nl ? a.codebook[tid] : 0.0f;   // first, so its LDS copy waits for it alone
  set_rows(s);
  load(0);   // in flight during the set-up below
  if (tid < 16) cb[tid] = cbv;
  // R^T: consecutive lanes take consecutive rows j of one 4-column slice, so
  // the transposed LDS writes fall in distinct banks
  for (int q = tid; q < D * D / 4; q += kTT) {
    const int j = q % D, k4 = q / D;
    const float4_t r = *(const float4_t *)(a.R + (int64_t)j * D + 4 * k4);
#pragma unroll
    for (int e = 0; e < 4; ++e) rt[(4 * k4 + e) * D + j] = r[e];
  }
  lds_barrier();
  build_cell_table<kTT>(cb, nl, tid, cells, thr, ucell, &table_ok);
  use_table = table_ok != 0;
  store_x(0);
  __syncthreads();
  for (; s < steps; s += gridDim.x) {
#pragma unroll
    for (int u = 0; u < VT; ++u)
#pragma unroll
      for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[u][g][i] = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const bool last = c == NC - 1;
      const bool have_next = !last || s + gridDim.x < steps;
      if (last && have_next) set_rows(s + gridDim.x);
      if (have_next) load(last ? 0 : c + 1);
      if (QJL && last) load_p(0);
      if (c == 0 && s != blockIdx.x) flush(s - gridDim.x);
      if (QJL && c == 1 && s != blockIdx.x) flush_signs(s - gridDim.x);
      compute(c & 1, c);
      if (last) quantise(s);
      if (have_next) store_x((c + 1) & 1);
      if (QJL && last) store_p(0);
      __syncthreads();
    }
    if constexpr (QJL) {
#pragma unroll
      for (int u = 0; u < VT; ++u)
#pragma unroll
        for (int g = 0; g < NG; ++g)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc2[u][g][i] = 0.0f;
#pragma unroll
      for (int pc = 0; pc < NPK; ++pc) {
        if (pc + 1 < NPK) load_p(pc + 1);
        project(pc & 1, pc);
        if (pc + 1 < NPK) store_p((pc + 1) & 1);
        __syncthreads();
      }
      signs();
    }
  }
  if constexpr (QJL) __syncthreads();   // the last step's sign bytes
  flush(s - gridDim.x);
  flush_signs(s - gridDim.x);
}

// The tiled encoder applies to inputs it can read in 16-byte pieces and
// outputs it can write in dwords: 16-byte aligned x rows, R and P_rot,
// 4-byte aligned blocks, signs and row strides (pages are 16-byte aligned by
// contract), fewer than 2^32 vectors.
bool tiled_encode_ok(const EncodeArgs &a, int x_dtype) {
  const int64_t es = x_dtype == 0 ? 4 : 2;
  const int64_t n = a.n_outer * a.n_inner;
  const bool qjl = a.qjl != nullptr || a.qjl_pages != nullptr;
  if (a.d != 64 && a.d != 128) return false;
  if (n <= 0 || n > ((int64_t)1 << 32) - 1024) return false;
  if ((uintptr_t)a.x % 16 || (uintptr_t)a.R % 16) return false;
  if (a.n_outer > 1 && (a.x_outer_stride * es) % 16) return false;
  if (a.pages == nullptr && ((uintptr_t)a.blocks % 4 || (a.n_outer > 1 && a.blocks_outer_stride % 4))) return false;
  if (qjl) {
    if (a.m != a.d || a.p_rot == nullptr || (uintptr_t)a.p_rot % 16) return false;
    if (a.qjl_pages == nullptr && ((uintptr_t)a.qjl % 4 || (a.n_outer > 1 && a.qjl_outer_stride % 4))) return false;
  }
  return true;
}

// Step size: the smallest halving (from min_sh, at most 2) whose steps give
// every compute unit one, so small launches spread over more compute units.
static int tiled_shift(int64_t n, int d, int min_sh) {
  const int full = d == 128 ? TiledShape<128, 0>::VS : TiledShape<64, 0>::VS;
  int sh = min_sh;
  while (sh < 2 && (n + (full >> sh) - 1) / (full >> sh) < device_compute_units()) ++sh;
  return sh;
}

static int tiled_grid(int64_t n, int d, int sh) {
  const int vs = (d == 128 ? TiledShape<128, 0>::VS : TiledShape<64, 0>::VS) >> sh;
  const int64_t steps = (n + vs - 1) / vs;
  const int64_t cap = device_compute_units();
  return (int)(steps < cap ? steps : cap);
}

hipError_t launch_encode_tiled(const EncodeArgs &a, int x_dtype, hipStream_t s) {
  const int64_t n = a.n_outer * a.n_inner;
  const int nl = 1 << a.bits;
  if (a.qjl != nullptr || a.qjl_pages != nullptr) {
    // QJL keys: half-size steps or smaller (LDS room for the residuals and P_rot)
    const int sh = tiled_shift(n, a.d, 1);
    const int grid = tiled_grid(n, a.d, sh);
#define PQKV_ETQ_T(DD, BB, TT)                                                                   \
  do {                                                                                           \
    if (sh == 1) encode_tiled_kernel<DD, BB, TT, 1, true><<<grid, kTT, 0, s>>>(a, nl, nullptr);  \
    else encode_tiled_kernel<DD, BB, TT, 2, true><<<grid, kTT, 0, s>>>(a, nl, nullptr);          \
  } while (0)
#define PQKV_ETQ(DD, BB)                              \
  do {                                                \
    if (x_dtype == 0) PQKV_ETQ_T(DD, BB, float);      \
    else if (x_dtype == 1) PQKV_ETQ_T(DD, BB, half_t); \
    else PQKV_ETQ_T(DD, BB, bf16_t);                  \
  } while (0)
    if (a.d == 128 && a.bits == 4) PQKV_ETQ(128, 4);
    else if (a.d == 128) PQKV_ETQ(128, 2);
    else if (a.bits == 4) PQKV_ETQ(64, 4);
    else PQKV_ETQ(64, 2);
#undef PQKV_ETQ
#undef PQKV_ETQ_T
    return hipGetLastError();
  }
  const int sh = tiled_shift(n, a.d, 0);
  const int grid = tiled_grid(n, a.d, sh);
#define PQKV_ET_T(DD, BB, TT)                                                             \
  do {                                                                                    \
    if (sh == 0) encode_tiled_kernel<DD, BB, TT, 0><<<grid, kTT, 0, s>>>(a, nl, nullptr); \
    else if (sh == 1) encode_tiled_kernel<DD, BB, TT, 1><<<grid, kTT, 0, s>>>(a, nl, nullptr); \
    else encode_tiled_kernel<DD, BB, TT, 2><<<grid, kTT, 0, s>>>(a, nl, nullptr);         \
  } while (0)
#define PQKV_ET(DD, BB)                          \
  do {                                           \
    if (x_dtype == 0) PQKV_ET_T(DD, BB, float);  \
    else if (x_dtype == 1) PQKV_ET_T(DD, BB, half_t); \
    else PQKV_ET_T(DD, BB, bf16_t);              \
  } while (0)
  if (a.d == 128 && a.bits == 4) PQKV_ET(128, 4);
  else if (a.d == 128) PQKV_ET(128, 2);
  else if (a.bits == 4) PQKV_ET(64, 4);
  else PQKV_ET(64, 2);
#undef PQKV_ET
#undef PQKV_ET_T
  return hipGetLastError();
}

bool tiled_soa_ok(const float *x, const float *R, const uint8_t *packed, int64_t n, int d) {
  return (d == 64 || d == 128) && n > 0 && n <= ((int64_t)1 << 32) - 1024 && (uintptr_t)x % 16 == 0 &&
         (uintptr_t)R % 16 == 0 && (uintptr_t)packed % 4 == 0;
}

hipError_t launch_encode_soa_tiled(const float *x, const float *R, const float *codebook, int n_levels,
                                   float *radius, uint8_t *packed, int64_t n, int d, hipStream_t s) {
  EncodeArgs a{};
  a.x = x;
  a.x_outer_stride = 0;
  a.R = R;
  a.codebook = codebook;
  a.blocks = packed;
  a.n_outer = 1;
  a.n_inner = n;
  a.d = d;
  const int sh = tiled_shift(n, d, 0);
  const int grid = tiled_grid(n, d, sh);
#define PQKV_ES(DD)                                                                                  \
  do {                                                                                               \
    if (sh == 0) encode_tiled_kernel<DD, 0, float, 0><<<grid, kTT, 0, s>>>(a, n_levels, radius);     \
    else if (sh == 1) encode_tiled_kernel<DD, 0, float, 1><<<grid, kTT, 0, s>>>(a, n_levels, radius); \
    else encode_tiled_kernel<DD, 0, float, 2><<<grid, kTT, 0, s>>>(a, n_levels, radius);             \
  } while (0)
  if (d == 128) PQKV_ES(128);
  else PQKV_ES(64);
#undef PQKV_ES
  return hipGetLastError();
}

}  // namespace pqkv
