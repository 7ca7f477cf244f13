// Expert-grouped GEMM on the MFMA cores, for batches of tokens (batched
// decode and prefill).
//
// Replaces the reference's prefill kernels (src/uma_qmoe/native/packed_q4_kernel.cu:560-776
// for Q4, :781-1099 for Q8; launchers :1486-1641) and its BF16 grouped_mm path
// (src/uma_qmoe/native_backend.py:958-1005), and serves the shared expert too.
//
// One workgroup = 4 waves computes an output block of (rows of one expert) x
// (one tile of up to 16*NB routes of that expert):
//   * weights go from HBM straight into MFMA A operands, each wave streaming
//     its own rows through a ring of in-flight 16-byte loads; Q4 nibbles and
//     Q8 bytes become exact bf16 integers (q + bias) in registers, so the
//     MFMA sums x*(q + bias) over one 128-element group and the epilogue
//     applies scale*(sum - bias*sum(x)) in FP32;
//   * the routes' activations are gathered into LDS 128 K-elements at a time
//     (double-buffered, prefetched one step ahead through registers) and read
//     as MFMA B operands by every wave;
//   * the 4 waves split the rows (WR = 4/KW row groups) and/or the K range
//     (KW groups, partial sums combined through LDS at the end); whole
//     workgroups can also split K (gridDim.y) and write FP32 partials that the
//     combine kernel adds.
// MFMA: v_mfma_f32_16x16x32_bf16. A lane l holds row l%16 / token l%16 and
// K-slice 8*(l/16)..+7 of A / B; D lane l holds token l%16, rows 4*(l/16)+i.
// The K elements a lane feeds each MFMA follow the order of its weight loads;
// A and B use the same order, so the sum is unchanged.
//
// Work tiles come from the device-built tile list (expert, first route); the
// linear workgroup id is remapped so that each XCD (id % 8) walks a
// contiguous range of (row block, tile) pairs with tiles fastest: the tiles
// of one hot expert reuse the same weight rows through that XCD's L2.
#include "uqm_internal.h"

namespace uqm {
namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

template <int ENC>
struct MEnc;
template <>
struct MEnc<kQ4> {
  static constexpr int kLoads = 1;        // 16-byte loads per lane per 128-element chunk
  static constexpr int kChunkBytes = 64;  // bytes of one row's 128-element chunk
  static constexpr float kBias = 136.0f;  // bf16(0x4300 | (nibble ^ 8)) = 136 + q
};
template <>
struct MEnc<kQ8> {
  static constexpr int kLoads = 2;
  static constexpr int kChunkBytes = 128;
  static constexpr float kBias = 128.0f;  // byte ^ 0x80 = q + 128
};
template <>
struct MEnc<kBF16> {
  static constexpr int kLoads = 4;
  static constexpr int kChunkBytes = 256;
  static constexpr float kBias = 0.0f;
};

constexpr int kChunk = 128;         // K elements per step
constexpr int kPitch = kChunk + 8;  // staged bf16 per token row; +16 B keeps ds_read_b128 conflict-free

__device__ __forceinline__ uint32_t dw(const uint4& v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

__device__ __forceinline__ uint32_t hi16_pair(float lo, float hi) {
  // bf16 halves of two floats that are exact in bf16 (integers 0..255).
  return perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// A operand (8 weights) of K-step S of a 128-element chunk.
//   Q4: dword S of the lane's 16-byte load = elements 32q+8S .. +7
//   Q8: load S/2, dwords 2(S%2), 2(S%2)+1 = elements 64(S/2)+16q+8(S%2) .. +7
//   BF16: load S = elements 32S+8q .. +7
template <int ENC, int S>
__device__ __forceinline__ bf16x8_t a_frag(const uint4 (&v)[MEnc<ENC>::kLoads]) {
  u32x4_t o;
  if constexpr (ENC == kQ4) {
    const uint32_t w = dw(v[0], S) ^ 0x88888888u;
    const uint32_t lo = w & 0x0F0F0F0Fu;
    const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;
    o.x = perm(hi, lo, 0x0C040C00u) | 0x43004300u;
    o.y = perm(hi, lo, 0x0C050C01u) | 0x43004300u;
    o.z = perm(hi, lo, 0x0C060C02u) | 0x43004300u;
    o.w = perm(hi, lo, 0x0C070C03u) | 0x43004300u;
  } else if constexpr (ENC == kQ8) {
    const uint32_t d0 = dw(v[S >> 1], 2 * (S & 1)) ^ 0x80808080u;
    const uint32_t d1 = dw(v[S >> 1], 2 * (S & 1) + 1) ^ 0x80808080u;
    o.x = hi16_pair(static_cast<float>(d0 & 0xFFu), static_cast<float>((d0 >> 8) & 0xFFu));
    o.y = hi16_pair(static_cast<float>((d0 >> 16) & 0xFFu), static_cast<float>(d0 >> 24));
    o.z = hi16_pair(static_cast<float>(d1 & 0xFFu), static_cast<float>((d1 >> 8) & 0xFFu));
    o.w = hi16_pair(static_cast<float>((d1 >> 16) & 0xFFu), static_cast<float>(d1 >> 24));
  } else {
    o.x = v[S].x;
    o.y = v[S].y;
    o.z = v[S].z;
    o.w = v[S].w;
  }
  return __builtin_bit_cast(bf16x8_t, o);
}

// Element offset (within a staged 128-element chunk) of the B operand of
// K-step S for lane quadrant q, matching a_frag's order.
template <int ENC, int S>
__device__ __forceinline__ int b_offset(int q) {
  if constexpr (ENC == kQ4) return 32 * q + 8 * S;
  else if constexpr (ENC == kQ8) return 64 * (S >> 1) + 16 * q + 8 * (S & 1);
  else return 32 * S + 8 * q;
}

template <int ENC, int AT, int NB, int S>
__device__ __forceinline__ void mfma_step(const uint4 (&w)[AT][MEnc<ENC>::kLoads], const uint16_t* xrow, int q,
                                          f32x4_t (&d)[AT][NB]) {
  bf16x8_t bfr[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b)
    bfr[b] = *reinterpret_cast<const bf16x8_t*>(xrow + b * 16 * kPitch + b_offset<ENC, S>(q));
#pragma unroll
  for (int ai = 0; ai < AT; ++ai) {
    const bf16x8_t af = a_frag<ENC, S>(w[ai]);
#pragma unroll
    for (int b = 0; b < NB; ++b) d[ai][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bfr[b], d[ai][b], 0, 0, 0);
  }
}

}  // namespace

template <int ENC, int NMAT, int RT, int NB, int KW, int MODE>
__global__ __launch_bounds__(256) void expert_mfma_kernel(MfmaArgs a) {
  using M = MEnc<ENC>;
  constexpr int L = M::kLoads;
  constexpr bool kScaled = ENC != kBF16;
  constexpr int AT = NMAT * RT;  // 16-row A tiles per wave
  constexpr int WR = 4 / KW;     // waves along rows
  constexpr int NTOK = 16 * NB;  // routes per tile
  constexpr int WGR = 16 * RT * WR;  // rows per workgroup (per matrix)
  constexpr int kRing = KW == 1 ? 16 : 8;                       // 16-byte weight loads in flight per lane
  constexpr int P = (kRing / (AT * L)) > 1 ? (kRing / (AT * L)) : 1;  // weight steps in flight per wave
  constexpr int NX = KW * NB;    // 16-byte activation loads per thread per step
  constexpr int kBufElems = KW * NTOK * kPitch;
  static_assert(KW == 1 || KW == 2 || KW == 4, "KW must divide the 4 waves");
  static_assert(NMAT == 1 || RT == 1, "gate/up tiles use one 16-row tile per matrix");

  extern __shared__ __align__(16) unsigned char lds[];
  uint16_t* xs = reinterpret_cast<uint16_t*>(lds);                          // [2][KW][NTOK][kPitch]
  float* xsum = reinterpret_cast<float*>(lds + 2 * kBufElems * 2);           // [2][KW][NTOK]
  float* scl = xsum + 2 * KW * NTOK;                                         // [NMAT][G][WGR]

  // ---- work tile (XCD-aware order: each XCD walks a contiguous range) ----
  const unsigned per_xcd = gridDim.x >> 3;
  const unsigned p = (blockIdx.x & 7u) * per_xcd + (blockIdx.x >> 3);
  if (p >= static_cast<unsigned>(a.row_blocks) * static_cast<unsigned>(a.tile_bound)) return;
  const int rblk = static_cast<int>(p / static_cast<unsigned>(a.tile_bound));
  const int tile = static_cast<int>(p % static_cast<unsigned>(a.tile_bound));
  int expert = 0, rbeg, nt;
  if (a.tiles != nullptr) {
    if (tile >= *a.tile_count) return;
    expert = a.tiles[2 * tile];
    rbeg = a.tiles[2 * tile + 1];
    nt = min(NTOK, a.expert_offsets[expert + 1] - rbeg);
  } else {
    rbeg = tile * NTOK;
    nt = min(NTOK, a.n_routes - rbeg);
  }
  if (nt <= 0) return;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int q = lane >> 4;
  const int wr = wave % WR;
  const int kw = wave / WR;

  const int nch = static_cast<int>(a.K / kChunk);
  const int cps = (nch + a.ksplit - 1) / a.ksplit;
  const int c_begin = blockIdx.y * cps;
  const int c_end = min(nch, c_begin + cps);
  if (c_begin >= c_end) return;  // uniform over the workgroup
  const int steps = (c_end - c_begin + KW - 1) / KW;
  const int G = kScaled ? static_cast<int>(a.K / a.group) : 0;  // scale groups per row
  const int gdiv = kScaled ? static_cast<int>(a.group / kChunk) : 1;

  const int64_t wg_row0 = static_cast<int64_t>(rblk) * WGR;
  const int64_t row_bytes = ENC == kQ4 ? a.K / 2 : (ENC == kQ8 ? a.K : 2 * a.K);

  // ---- per-lane weight pointers (A layout: row lane%16, 16-byte slot q) ----
  const uint8_t* wp[AT];
#pragma unroll
  for (int ai = 0; ai < AT; ++ai) {
    const int m = NMAT == 2 ? ai : 0;
    const int rt = NMAT == 2 ? 0 : ai;
    const int64_t row = wg_row0 + wr * 16 * RT + rt * 16 + (lane & 15);
    wp[ai] = a.w[m] + (static_cast<int64_t>(expert) * a.rows + row) * row_bytes + q * 16;
  }

  // ---- scales of the workgroup's rows into LDS, transposed to [m][g][row] ----
  if constexpr (kScaled) {
    for (int idx = tid; idx < NMAT * WGR * G; idx += 256) {
      const int g = idx % G;
      const int rr = (idx / G) % WGR;
      const int m = idx / (G * WGR);
      scl[(m * G + g) * WGR + rr] =
          a.s[m][static_cast<int64_t>(expert) * a.scales_per_expert + (wg_row0 + rr) * G + g];
    }
  }

  // ---- activation rows this thread stages (fixed over the K loop) ----
  const uint16_t* xp[NX];
  bool xv[NX];
#pragma unroll
  for (int i = 0; i < NX; ++i) {
    const int idx = tid + 256 * i;
    const int tok = (idx >> 4) % NTOK;
    xv[i] = tok < nt;
    int route = rbeg + (xv[i] ? tok : 0);
    if (a.route_order != nullptr) route = a.route_order[route];
    xp[i] = a.x + static_cast<int64_t>(route / a.x_div) * a.ldx + (idx & 15) * 8;
  }
  auto load_x = [&](int j, uint4 (&r)[NX]) {
#pragma unroll
    for (int i = 0; i < NX; ++i) {
      const int kwi = ((tid + 256 * i) >> 4) / NTOK;
      const int c = c_begin + j * KW + kwi;
      r[i] = (xv[i] && c < c_end) ? ldg16(xp[i] + static_cast<int64_t>(c) * kChunk) : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_x = [&](int buf, const uint4 (&r)[NX]) {
#pragma unroll
    for (int i = 0; i < NX; ++i) {
      const int idx = tid + 256 * i;
      const int rowid = idx >> 4;  // kwi * NTOK + tok
      *reinterpret_cast<uint4*>(xs + buf * kBufElems + rowid * kPitch + (idx & 15) * 8) = r[i];
      if constexpr (kScaled) {
        float s = bf16lo(r[i].x) + bf16hi(r[i].x) + bf16lo(r[i].y) + bf16hi(r[i].y) + bf16lo(r[i].z) +
                  bf16hi(r[i].z) + bf16lo(r[i].w) + bf16hi(r[i].w);
        s += xor_partner<8>(s);
        s += xor_partner<4>(s);
        s += xor_partner<2>(s);
        s += xor_partner<1>(s);
        if ((idx & 15) == 0) xsum[buf * KW * NTOK + rowid] = s;
      }
    }
  };

  // ---- weight ring ----
  uint4 ring[P][AT][L];
  auto load_w = [&](int j, uint4 (&slot)[AT][L]) {
    const int c = c_begin + j * KW + kw;
    if (c < c_end) {
#pragma unroll
      for (int ai = 0; ai < AT; ++ai)
#pragma unroll
        for (int u = 0; u < L; ++u)
          slot[ai][u] = ldg16(wp[ai] + static_cast<int64_t>(c) * M::kChunkBytes + u * 64);
    }
  };

  f32x4_t acc[AT][NB];
#pragma unroll
  for (int ai = 0; ai < AT; ++ai)
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[ai][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int j = 0; j < P; ++j)
    if (j < steps) load_w(j, ring[j]);
  uint4 xr[NX];
  load_x(0, xr);
  store_x(0, xr);
  if (steps > 1) load_x(1, xr);
  __syncthreads();

  for (int j0 = 0; j0 < steps; j0 += P) {
#pragma unroll
    for (int jj = 0; jj < P; ++jj) {
      const int j = j0 + jj;
      if (j >= steps) break;
      const int buf = j & 1;
      const int c = c_begin + j * KW + kw;
      if (c < c_end) {
        const uint16_t* xrow = xs + buf * kBufElems + (kw * NTOK + (lane & 15)) * kPitch;
        if constexpr (kScaled) {
          f32x4_t d[AT][NB];
#pragma unroll
          for (int ai = 0; ai < AT; ++ai)
#pragma unroll
            for (int b = 0; b < NB; ++b) d[ai][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
          mfma_step<ENC, AT, NB, 0>(ring[jj], xrow, q, d);
          mfma_step<ENC, AT, NB, 1>(ring[jj], xrow, q, d);
          mfma_step<ENC, AT, NB, 2>(ring[jj], xrow, q, d);
          mfma_step<ENC, AT, NB, 3>(ring[jj], xrow, q, d);
          const int g = c / gdiv;
          float xsv[NB];
#pragma unroll
          for (int b = 0; b < NB; ++b) xsv[b] = M::kBias * xsum[buf * KW * NTOK + kw * NTOK + b * 16 + (lane & 15)];
#pragma unroll
          for (int ai = 0; ai < AT; ++ai) {
            const int m = NMAT == 2 ? ai : 0;
            const int rt = NMAT == 2 ? 0 : ai;
            const float4 sc =
                *reinterpret_cast<const float4*>(scl + (m * G + g) * WGR + wr * 16 * RT + rt * 16 + 4 * q);
#pragma unroll
            for (int b = 0; b < NB; ++b) {
              acc[ai][b][0] = fmaf(sc.x, d[ai][b][0] - xsv[b], acc[ai][b][0]);
              acc[ai][b][1] = fmaf(sc.y, d[ai][b][1] - xsv[b], acc[ai][b][1]);
              acc[ai][b][2] = fmaf(sc.z, d[ai][b][2] - xsv[b], acc[ai][b][2]);
              acc[ai][b][3] = fmaf(sc.w, d[ai][b][3] - xsv[b], acc[ai][b][3]);
            }
          }
        } else {
          mfma_step<ENC, AT, NB, 0>(ring[jj], xrow, q, acc);
          mfma_step<ENC, AT, NB, 1>(ring[jj], xrow, q, acc);
          mfma_step<ENC, AT, NB, 2>(ring[jj], xrow, q, acc);
          mfma_step<ENC, AT, NB, 3>(ring[jj], xrow, q, acc);
        }
      }
      if (j + P < steps) load_w(j + P, ring[jj]);
      if (j + 1 < steps) {
        store_x(buf ^ 1, xr);
        if (j + 2 < steps) load_x(j + 2, xr);
      }
      __syncthreads();
    }
  }

  // ---- combine the K groups of waves ----
  if constexpr (KW > 1) {
    float* red = reinterpret_cast<float*>(lds);
    constexpr int kVals = AT * NB * 4;
    if (kw > 0) {
#pragma unroll
      for (int ai = 0; ai < AT; ++ai)
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            red[(((kw - 1) * WR + wr) * kVals + (ai * NB + b) * 4 + i) * 64 + lane] = acc[ai][b][i];
    }
    __syncthreads();
    if (kw != 0) return;
#pragma unroll
    for (int o = 1; o < KW; ++o)
#pragma unroll
      for (int ai = 0; ai < AT; ++ai)
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            acc[ai][b][i] += red[(((o - 1) * WR + wr) * kVals + (ai * NB + b) * 4 + i) * 64 + lane];
  }

  // ---- epilogue: D lane holds token lane%16 of each B tile, rows 4q..4q+3 ----
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int tok = b * 16 + (lane & 15);
    if (tok >= nt) continue;
    int route = rbeg + tok;
    if (a.route_order != nullptr) route = a.route_order[route];
    if constexpr (MODE == kModeSilu) {
      const int64_t r0 = wg_row0 + wr * 16 + 4 * q;
      uint16_t h[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) h[i] = f32_to_bf16(silu(round_bf16(acc[0][b][i])) * round_bf16(acc[1][b][i]));
      const uint2 v = make_uint2(static_cast<uint32_t>(h[0]) | (static_cast<uint32_t>(h[1]) << 16),
                                 static_cast<uint32_t>(h[2]) | (static_cast<uint32_t>(h[3]) << 16));
      *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(a.out) + static_cast<int64_t>(route) * a.ldo + r0) = v;
    } else {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const int64_t r0 = wg_row0 + wr * 16 * RT + rt * 16 + 4 * q;
        float* dst = reinterpret_cast<float*>(a.out) + blockIdx.y * a.part_stride + static_cast<int64_t>(route) * a.ldo + r0;
        *reinterpret_cast<float4*>(dst) = make_float4(acc[rt][b][0], acc[rt][b][1], acc[rt][b][2], acc[rt][b][3]);
      }
    }
  }
}

namespace {

template <int ENC, int NMAT, int RT, int NB, int KW>
size_t lds_bytes_for(int64_t K, int64_t group) {
  constexpr int NTOK = 16 * NB;
  const size_t xs = 2ull * KW * NTOK * kPitch * 2 + 2ull * KW * NTOK * 4;
  const size_t G = ENC == kBF16 ? 0 : static_cast<size_t>(K / group);
  return xs + sizeof(float) * NMAT * G * (16 * RT * (4 / KW));
}

template <int ENC, int NMAT, int RT, int NB, int KW>
hipError_t launch_cfg(const MfmaArgs& args, hipStream_t stream) {
  constexpr int WGR = 16 * RT * (4 / KW);
  MfmaArgs a = args;
  a.row_blocks = static_cast<int32_t>(a.rows / WGR);
  const size_t lds = lds_bytes_for<ENC, NMAT, RT, NB, KW>(a.K, a.group);
  if (lds > 160 * 1024) return hipErrorInvalidValue;
  const unsigned total = static_cast<unsigned>(a.row_blocks) * static_cast<unsigned>(a.tile_bound);
  const unsigned grid = (total + 7u) & ~7u;
  constexpr int MODE = NMAT == 2 ? kModeSilu : kModeF32;
  auto kernel = expert_mfma_kernel<ENC, NMAT, RT, NB, KW, MODE>;
  if (lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kernel, dim3(grid, static_cast<unsigned>(a.ksplit)), dim3(256), lds, stream, a);
  return hipGetLastError();
}

template <int ENC, int NMAT, int RT, int KW>
hipError_t launch_nb(const MfmaArgs& a, int nb, hipStream_t stream) {
  if (nb <= 1) return launch_cfg<ENC, NMAT, RT, 1, KW>(a, stream);
  if (nb <= 2) return launch_cfg<ENC, NMAT, RT, 2, KW>(a, stream);
  if constexpr (KW == 1) {
    if (nb <= 4 || ENC != kBF16) return launch_cfg<ENC, NMAT, RT, 4, KW>(a, stream);
    if constexpr (ENC == kBF16) return launch_cfg<ENC, NMAT, RT, 8, KW>(a, stream);
  }
  return hipErrorInvalidValue;
}

template <int ENC>
hipError_t launch_enc(int nmat, const MfmaArgs& a, int nb, int kw, int rt, hipStream_t stream) {
  if (nmat == 2) {
    if (kw == 4) return launch_nb<ENC, 2, 1, 4>(a, nb, stream);
    return launch_nb<ENC, 2, 1, 1>(a, nb, stream);
  }
  if (kw == 4) return launch_nb<ENC, 1, 1, 4>(a, nb, stream);
  if (rt == 2) return launch_nb<ENC, 1, 2, 1>(a, nb, stream);
  return launch_nb<ENC, 1, 1, 1>(a, nb, stream);
}

}  // namespace

bool mfma_supported(int enc, int64_t rows, int64_t K, int64_t group) {
  if (rows <= 0 || rows % 64 != 0 || K <= 0 || K % kChunk != 0) return false;
  if (enc == kBF16) return true;
  return group > 0 && group % kChunk == 0 && K % group == 0 && K / group <= 64;
}

hipError_t launch_expert_mfma(int enc, int nmat, const MfmaArgs& args, int nb, int kw, int rt, hipStream_t stream) {
  MfmaArgs a = args;
  if (a.ksplit < 1) a.ksplit = 1;
  if (nmat == 2 && a.ksplit != 1) return hipErrorInvalidValue;
  if (kw != 1 && kw != 4) return hipErrorInvalidValue;
  if (kw == 4 && nb > 2) return hipErrorInvalidValue;
  const int wgr = 16 * (nmat == 2 ? 1 : rt) * (4 / kw);
  if (a.rows % wgr != 0) return hipErrorInvalidValue;
  if (enc != kBF16) a.scales_per_expert = (a.rows * a.K + a.group - 1) / a.group;
  if (a.tile_bound <= 0) return hipSuccess;
  if (enc == kQ4) return launch_enc<kQ4>(nmat, a, nb, kw, rt, stream);
  if (enc == kQ8) return launch_enc<kQ8>(nmat, a, nb, kw, rt, stream);
  return launch_enc<kBF16>(nmat, a, nb, kw, rt, stream);
}

}  // namespace uqm
