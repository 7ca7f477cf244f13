// Expert-grouped GEMM on the MFMA cores, for batches of tokens (batched
// decode and prefill).
//
// Replaces the reference's prefill kernels (src/uma_qmoe/native/packed_q4_kernel.cu:560-776
// for Q4, :781-1099 for Q8; launchers :1486-1641) and its BF16 grouped_mm path
// (src/uma_qmoe/native_backend.py:958-1005), and serves the shared expert too.
//
// One workgroup computes an output block of (rows of one expert) x (one tile
// of up to 16*NB routes of that expert). It is split into producer and
// consumer waves:
//   * NL loader waves move every byte the step needs from global memory into
//     LDS with global_load_lds (16 bytes per lane, no registers): the weight
//     rows of the MMA waves and the gathered activations of the tile, for
//     D steps ahead (a ring of D LDS buffers). Their only waits are their own
//     vmcnt waits for the step about to be consumed, so the weight stream is
//     never serialised behind anything else;
//   * MW MMA waves (4 or 8) read A (weights) and B (activations) fragments from LDS and
//     issue v_mfma_f32_16x16x32_bf16. Q4 nibbles and Q8 bytes become exact
//     bf16 integers (q + bias) in registers, the MFMA sums x * (q + bias) over
//     one 128-element scale group, and the epilogue applies
//     scale * (sum - bias * sum(x)) in FP32 (sum(x) comes from one more MFMA
//     of the same B fragments with a ones-matrix). BF16 weights accumulate
//     directly.
// One s_barrier per step hands buffers between the two sides.
//
// The MMA waves split the rows (WR = MW/KW row groups) and/or the K range
// (KW groups, partial sums combined through LDS at the end); whole workgroups
// can also split K (gridDim.y) and write FP32 partials the combine kernel adds.
//
// MFMA operand layout (v_mfma_f32_16x16x32_bf16): A lane l holds row l%16 and
// K-slice 8*(l/16)..+7; B lane l holds token l%16, same K-slice; D lane l
// holds token l%16, rows 4*(l/16)+i. The K elements a lane feeds each MFMA
// follow the order of its 16-byte weight slots; A and B use the same order,
// so the sum is unchanged. Activation rows are stored in LDS with their
// 16-byte slots reordered (the slot a lane of quadrant q reads at K-step S
// sits at position q + 4 S) and XOR-swizzled by the token index, so the B
// reads of all 64 lanes hit distinct banks (b_position).
//
// Q4 gate/up tiles of 16 routes also have a wide form (kQ4Wide): a step
// covers two 128-element scale groups, 128 contiguous bytes of a row, and each
// 1 KB weight load takes 8 rows x 128 B instead of 16 rows x 64 B. A lane then
// fills the 16 bytes of one row segment (XOR-swizzled by the row so that the
// MMA waves' A reads are free of bank conflicts) and an MMA lane reads two of
// them, one per scale group. Loads of 128-byte row segments stream faster than
// loads of 64-byte ones (device-wide, through LDS DMA: 6.0-6.2 vs 5.6-5.7
// TB/s); the batch-32 gate/up kernel takes 45.5 vs 48.6 us (kernel trace).
//
// Work tiles come from the device-built tile list (expert, first route).
#include <atomic>
#include <type_traits>

#include "uqm_internal.h"

namespace uqm {
namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) unsigned char lds_uchar_t;

// Q4 weights with two scale groups per step (kernel template value only; the
// weights are the same UQM_Q4 bytes)
constexpr int kQ4Wide = 3;

template <int ENC>
struct MEnc;
template <>
struct MEnc<kQ4> {
  static constexpr int kChunk = 128;      // K elements per step (one scale group)
  static constexpr int kLoads = 1;        // 16-byte slots per lane per step and A tile
  static constexpr int kChunkBytes = 64;  // bytes of one row's chunk
  static constexpr int kBits = 4;         // bits per weight
  static constexpr float kBias = 136.0f;  // bf16(0x4300 | (nibble ^ 8)) = 136 + q
};
template <>
struct MEnc<kQ4Wide> {
  static constexpr int kChunk = 256;
  static constexpr int kLoads = 2;
  static constexpr int kChunkBytes = 128;
  static constexpr int kBits = 4;
  static constexpr float kBias = 136.0f;
};
template <>
struct MEnc<kQ8> {
  static constexpr int kChunk = 128;
  static constexpr int kLoads = 2;
  static constexpr int kChunkBytes = 128;
  static constexpr int kBits = 8;
  static constexpr float kBias = 128.0f;  // byte ^ 0x80 = q + 128
};
template <>
struct MEnc<kBF16> {
  static constexpr int kChunk = 64;
  static constexpr int kLoads = 2;
  static constexpr int kChunkBytes = 128;
  static constexpr int kBits = 16;
  static constexpr float kBias = 0.0f;
};

__device__ __forceinline__ uint32_t dw(const uint4& v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

__device__ __forceinline__ uint32_t hi16_pair(float lo, float hi) {
  // bf16 halves of two floats that are exact in bf16 (integers 0..255).
  return perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// A operand (8 weights) of K-step S of a chunk from the lane's 16-byte slots.
//   Q4: dword S%4 of slot S/4 = elements 128(S/4)+32q+8(S%4) .. +7 (one slot,
//       S < 4, in the narrow form)
//   Q8: slot S/2, dwords 2(S%2), 2(S%2)+1 = elements 64(S/2)+16q+8(S%2) .. +7
//   BF16: slot S = elements 32S+8q .. +7
template <int ENC, int S>
__device__ __forceinline__ bf16x8_t a_frag(const uint4 (&v)[MEnc<ENC>::kLoads]) {
  u32x4_t o;
  if constexpr (ENC == kQ4 || ENC == kQ4Wide) {
    // pair d = (element 2d, element 2d + 1) = low and high nibble of byte d:
    // v_perm puts byte d of w at bits 0-7 and byte d of w >> 4 at bits 16-23,
    // then one masked xor/or (a single v_bitop3) makes both bf16 values
    const uint32_t w = dw(v[S >> 2], S & 3);
    const uint32_t h = w >> 4;
    o.x = (perm(h, w, 0x0C040C00u) ^ 0x00080008u) & 0x000F000Fu | 0x43004300u;
    o.y = (perm(h, w, 0x0C050C01u) ^ 0x00080008u) & 0x000F000Fu | 0x43004300u;
    o.z = (perm(h, w, 0x0C060C02u) ^ 0x00080008u) & 0x000F000Fu | 0x43004300u;
    o.w = (perm(h, w, 0x0C070C03u) ^ 0x00080008u) & 0x000F000Fu | 0x43004300u;
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

// 16-byte slot (8 elements, within a chunk) of the B operand of K-step S for
// lane quadrant q, matching a_frag's order.
template <int ENC>
__device__ __forceinline__ int b_slot(int q, int S) {
  if constexpr (ENC == kQ4 || ENC == kQ4Wide) return 16 * (S >> 2) + 4 * q + (S & 3);
  else if constexpr (ENC == kQ8) return 8 * (S >> 1) + 2 * q + (S & 1);
  else return 4 * S + q;
}

// LDS position of that slot in a staged activation row: q + 4 S, XOR-ed with
// the row's token index (its low bits, up to 4). Reads of one K-step then have
// q in the low two bits of the position, which the gfx950 LDS serves without
// bank conflicts for all 64 lanes; with q in bits 2-3 (the chunk order of a Q4
// fragment) half of the LDS cycles of the batch-32 Q4 kernels were
// bank-conflict stalls (rocprofv3 SQ_LDS_BANK_CONFLICT), and a probe of both
// patterns on their own confirms it.
__device__ __forceinline__ int b_position(int q, int S, int row, int spr) {
  return (q + 4 * S) ^ (row & ((spr < 16 ? spr : 16) - 1));
}

// Weight loads: load u of a 16-row A tile puts lane l's 16 bytes at LDS byte
// 1024 u + 16 l of the tile. Row (within the tile) and byte (within the row's
// chunk) lane l loads there:
//   narrow: row l % 16, byte 16 (l / 16) + 64 u (16 rows x 64 B per load)
//   Q4 wide: row 8 u + l / 8, 16-byte segment (l % 8) ^ ((row / 2) % 8)
//            (8 rows x 128 B per load; the tile is row-major, 128 B per row)
template <int ENC>
__device__ __forceinline__ int a_load_row(int lane, int u) {
  if constexpr (ENC == kQ4Wide) return 8 * u + (lane >> 3);
  else return lane & 15;
}
template <int ENC>
__device__ __forceinline__ int a_load_byte(int lane, int u) {
  if constexpr (ENC == kQ4Wide) return 16 * ((lane & 7) ^ ((a_load_row<ENC>(lane, u) >> 1) & 7));
  else return 16 * (lane >> 4) + 64 * u;
}
// LDS byte (within the tile) of the MMA lane's slot u: narrow, the 16 bytes
// load u put there for this lane; Q4 wide, row l % 16's segment 4 u + l / 16
// (scale group u), where the swizzle put it. Lanes l and l + 16 k read rows
// l % 16 at distinct 16-byte bank groups.
template <int ENC>
__device__ __forceinline__ int a_read_off(int lane, int u) {
  if constexpr (ENC == kQ4Wide) {
    const int r = lane & 15;
    return 128 * r + 16 * ((4 * u + (lane >> 4)) ^ ((r >> 1) & 7));
  } else {
    return 1024 * u + 16 * lane;
  }
}

// s_waitcnt with only vmcnt limited (gfx9 encoding: vmcnt bits 3:0 and 15:14).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Waits until at most n * PER loads are outstanding (n < NMAX, wave-uniform).
template <int PER, int NMAX>
__device__ __forceinline__ void wait_vmcnt_steps(int n) {
  if constexpr (NMAX > 1) {
    if (n >= NMAX - 1) {
      wait_vmcnt<(NMAX - 1) * PER>();
      return;
    }
    wait_vmcnt_steps<PER, NMAX - 1>(n);
  } else {
    wait_vmcnt<0>();
  }
}

__device__ __forceinline__ void dma16(const void* src, void* lds_dst) {
  __builtin_amdgcn_global_load_lds(src, (lds_void_t*)(lds_dst), 16, 0, 0);
}

// Same, with the LDS destination as a (wave-uniform) LDS byte address.
__device__ __forceinline__ void dma16_to(const void* src, uint32_t lds_addr) {
  __builtin_amdgcn_global_load_lds(src, reinterpret_cast<lds_void_t*>(static_cast<uintptr_t>(lds_addr)), 16, 0, 0);
}

}  // namespace

template <int ENC, int NMAT, int MW, int NB, int KW>
struct MfmaCfg {
  using M = MEnc<ENC>;
  static constexpr int CH = M::kChunk;
  static constexpr int L = M::kLoads;
  static constexpr int KS = CH / 32;  // MFMA K-steps per chunk
  static constexpr int GPC = ENC == kQ4Wide ? 2 : 1;  // 128-element scale groups per step
  static constexpr int AT = NMAT;     // 16-row A tiles per MMA wave (gate and up, or one)
  static constexpr int WR = MW / KW;  // MMA waves along the rows
  static constexpr int NTOK = 16 * NB;
  static constexpr int WGR = 16 * WR;  // rows per work item (per matrix)
  static constexpr int ROWB = CH * 2;       // bytes of one staged activation row
  static constexpr int SPR = ROWB / 16;     // 16-byte slots per activation row
  static constexpr int W_BYTES = MW * AT * L * 1024;
  static constexpr int X_BYTES = KW * NTOK * ROWB;
  static constexpr int BUF = W_BYTES + X_BYTES;
  static constexpr int W_INSTR = MW * AT * L;  // 1 KB loads per step
  static constexpr int X_INSTR = X_BYTES / 1024;
  static constexpr int I_STEP = W_INSTR + X_INSTR;
  // ring depth: 48-route gate/up tiles (28 KB steps) keep 3 buffers so that
  // the ring, three scale slots and the metadata fit the 160 KB of LDS. The
  // Q4 down projection keeps two workgroups (two loader waves) per CU: its
  // 16-route tiles (12 KB steps) with 4 buffers (batch 32 100.6-100.8 vs
  // 102.3-102.5 us per call with 6, T = 16 80.0-80.3 vs 82.4-82.8), its
  // 48-route tiles (20 KB steps) with 3 buffers and two scale slots (c4
  // 166.7-167.2 vs 169.6-170.2 us with 4 buffers and three slots)
  static constexpr bool kDownPair = ENC == kQ4 && NMAT == 1 && NB == 1 && KW == 1 && MW == 8;
  static constexpr bool kDown48Pair = ENC == kQ4 && NMAT == 1 && NB == 3 && KW == 1 && MW == 8;
  static constexpr int D = kDownPair ? 4
                                     : (kDown48Pair ? 3 : (BUF <= 12 * 1024 ? 6
                                                         : (BUF <= 24 * 1024 || (BUF <= 32 * 1024 && NB != 3) ? 4 : 3)));
  static constexpr int NL = (D - 2) * I_STEP > 63 ? 2 : 1;  // loader waves
  static constexpr int I_WAVE = I_STEP / NL;
  static constexpr int THREADS = 64 * (MW + NL);
  // item slots for the scales: 2 for the wide Q4 gate/up tiles (40 KB steps),
  // whose ring and three slots would not fit the LDS, and for the Q4 down
  // projection's 48-route tiles (two workgroups per CU)
  static constexpr int SLOTS = (ENC == kQ4Wide && NMAT == 2) || kDown48Pair ? 2 : 3;
  static constexpr int MAX_ITEMS = NTOK <= 32 ? 32 : 16;  // work items per workgroup
  static constexpr int META = 4 + NTOK;                // expert, first route, routes, row block, route ids
  static constexpr int RED_BYTES = KW > 1 ? (KW - 1) * WR * AT * NB * 4 * 64 * 4 : 0;
  static constexpr int FIXED_LDS = D * BUF + RED_BYTES + MAX_ITEMS * META * 4;
  static_assert(W_INSTR % NL == 0 && X_INSTR % NL == 0, "loader waves share the step's loads evenly");
  static_assert((D - 2) * I_WAVE <= 63, "outstanding loads per loader wave must fit vmcnt");
  static_assert(X_BYTES % 1024 == 0, "activation tile must be whole 1 KB loads");
  static_assert(D * BUF <= 144 * 1024, "LDS ring too large");
};

// Persistent workgroups: the (row block, route tile) work items are split into
// 8 contiguous ranges, one per XCD (blockIdx % 8), and each XCD's range is
// dealt out round robin over its workgroups. With tiles fastest, the tiles of
// one expert (or of the shared expert) that share a row block run at the same
// time on neighbouring workgroups of one XCD, which read its weight rows once
// from HBM and share them through that XCD's L2 (c4: 205 vs 217 us per call
// with contiguous runs per workgroup, whose second pass over a row block found
// it evicted; c5 76 vs 79 us). With row blocks fastest, the row blocks of one
// tile run together and share its gathered activations instead, and each
// XCD reads only its own tiles' activations: the routed down projection's
// per-route inputs are larger than an XCD's L2 (c4 5.8 MB), which tiles
// fastest fetched from HBM by every XCD (c4 down 192 vs 99 MB per call for
// 92 MB of weights, c5 60 vs 28 MB for 20 MB). A workgroup loads the metadata of
// all its items into LDS once; after that its loader waves stream the items'
// steps back to back through the LDS ring, and the MMA waves write each
// item's outputs when its last step is done.
template <int ENC, int NMAT, int MW, int NB, int KW, int MODE>
__global__ __launch_bounds__((MfmaCfg<ENC, NMAT, MW, NB, KW>::THREADS)) void expert_mfma_kernel(MfmaArgs a) {
  using C = MfmaCfg<ENC, NMAT, MW, NB, KW>;
  constexpr int RT = 1;
  using M = typename C::M;
  constexpr int CH = C::CH, L = C::L, KS = C::KS, AT = C::AT, WR = C::WR, NTOK = C::NTOK, WGR = C::WGR;
  constexpr int D = C::D, NL = C::NL, SLOTS = C::SLOTS, META = C::META;
  constexpr bool kScaled = ENC != kBF16;
  static_assert(MW % KW == 0, "KW must divide the MMA waves");

  extern __shared__ __align__(16) unsigned char lds[];
  float* red = reinterpret_cast<float*>(lds + D * C::BUF);
  int* meta = reinterpret_cast<int*>(lds + D * C::BUF + C::RED_BYTES);
  float* scl = reinterpret_cast<float*>(meta + C::MAX_ITEMS * META);  // [SLOTS][NMAT][WGR][G]

  // ---- this workgroup's run of work items ----
  const int n_tiles = a.tiles != nullptr ? *a.tile_count : a.tile_bound;
  const int n_items = a.row_blocks * n_tiles;
  const int xcd = static_cast<int>(blockIdx.x & 7u);
  const int per = static_cast<int>(gridDim.x >> 3);
  const int wslot = static_cast<int>(blockIdx.x >> 3);
  const int xb = static_cast<int>(static_cast<int64_t>(n_items) * xcd / 8);
  const int xe = static_cast<int>(static_cast<int64_t>(n_items) * (xcd + 1) / 8);
  // this workgroup's items: xb + wslot + j * per (the launcher sizes the grid
  // so that a workgroup gets at most MAX_ITEMS)
  const int mine = xe - xb - wslot;
  const int nit = mine > 0 ? min((mine + per - 1) / per, C::MAX_ITEMS) : 0;
  if (nit <= 0) return;

  const int nch = static_cast<int>(a.K / CH);
  const int cps = (nch + a.ksplit - 1) / a.ksplit;
  const int c_begin = blockIdx.y * cps;
  const int c_end = min(nch, c_begin + cps);
  if (c_begin >= c_end) return;  // uniform over the workgroup
  const int S = (c_end - c_begin + KW - 1) / KW;  // steps per item
  const int total = nit * S;
  const int G = kScaled ? static_cast<int>(a.K / a.group) : 0;  // scale groups per row
  const int gdiv = kScaled ? static_cast<int>(a.group / 128) : 1;  // 128-element sub-chunks per scale group
  const int64_t row_bytes = a.K * M::kBits / 8;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;

  // ---- metadata of the run into LDS (every wave takes part in the barriers) ----
  bool row_fastest = a.order == kOrderRowFastest;
  if (a.order == kOrderAuto && a.tiles != nullptr && a.active_count != nullptr)
    row_fastest = 2 * n_tiles < 3 * *a.active_count;
  for (int i = tid; i < nit; i += C::THREADS) {
    const int item = xb + wslot + i * per;
    const int tile = row_fastest ? item / a.row_blocks : item % n_tiles;
    int expert = 0, rbeg, nt;
    if (a.tiles != nullptr) {
      expert = a.tiles[2 * tile];
      rbeg = a.tiles[2 * tile + 1];
      nt = min(NTOK, a.expert_offsets[expert + 1] - rbeg);
    } else {
      rbeg = tile * NTOK;
      nt = min(NTOK, a.n_routes - rbeg);
    }
    int* m = meta + i * META;
    m[0] = expert;
    m[1] = rbeg;
    m[2] = nt;
    m[3] = row_fastest ? item % a.row_blocks : item / n_tiles;
  }
  __syncthreads();
  for (int idx = tid; idx < nit * NTOK; idx += C::THREADS) {
    const int i = idx / NTOK;
    const int tok = idx - i * NTOK;
    int* m = meta + i * META;
    int route = m[1] + (tok < m[2] ? tok : 0);
    if (a.route_order != nullptr) route = a.route_order[route];
    m[4 + tok] = route;
  }
  __syncthreads();

  if (wave >= MW) {
    // =========================== loader waves ===========================
    const int lw = NL == 1 ? 0 : wave - MW;
    constexpr int XW = C::X_INSTR / NL;  // activation loads of this wave per step
    const uint8_t* wrow[AT][L];  // this lane's bytes of load u of A tile ai of MMA wave 0 (chunk 0 of the item)
    const uint8_t* xsrc[XW];     // this lane's activation row slot of each of its activation loads
    int xkw[XW];                 // K group of the chunk an activation load feeds
    int cur = -1;
    auto setup_item = [&](int i) {
      const int* m = meta + i * META;
      const int expert = m[0];
      const int64_t row0 = static_cast<int64_t>(m[3]) * WGR;
#pragma unroll
      for (int ai = 0; ai < AT; ++ai) {
        const int mat = NMAT == 2 ? ai : 0;
#pragma unroll
        for (int u = 0; u < L; ++u) {
          int64_t row = row0 + a_load_row<ENC>(lane, u);
          const int byte = a_load_byte<ENC>(lane, u);
          if constexpr (WR == 1) {
            // clamped padding rows and the appended tail row (router + shared-expert gate)
            if (a.rows_valid > 0 && row >= a.rows_valid) row = a.rows_valid - 1;
            if (mat == 0 && a.w_tail != nullptr && row >= a.tail_from) {
              wrow[ai][u] = a.w_tail + (row - a.tail_from) * row_bytes + byte;
              continue;
            }
          }
          wrow[ai][u] = a.w[mat] + (static_cast<int64_t>(expert) * a.rows + row) * row_bytes + byte;
        }
      }
#pragma unroll
      for (int k = 0; k < XW; ++k) {
        const int xi = k * NL + lw;
        const int r = xi * (1024 / C::ROWB) + lane / C::SPR;  // staged row = kwi * NTOK + tok
        const int tok = r % NTOK;
        // this lane fills LDS position lane % SPR of row r: the slot whose
        // (q, S) b_position maps there
        const int u = (lane % C::SPR) ^ (r & ((C::SPR < 16 ? C::SPR : 16) - 1));
        const int slot = b_slot<ENC>(u & 3, u >> 2);
        const int route = m[4 + tok];
        xsrc[k] = reinterpret_cast<const uint8_t*>(a.x + static_cast<int64_t>(route / a.x_div) * a.ldx) + slot * 16;
        xkw[k] = r / NTOK;
      }
      if constexpr (kScaled) {
        // the item's scales: per matrix one contiguous block of WGR rows x G groups
        if (lw == 0) {
          const int bytes = WGR * G * 4;
          unsigned char* dst = reinterpret_cast<unsigned char*>(scl + (i % SLOTS) * NMAT * WGR * G);
          for (int mat = 0; mat < NMAT; ++mat) {
            const uint8_t* s_src =
                reinterpret_cast<const uint8_t*>(a.s[mat] + static_cast<int64_t>(expert) * a.scales_per_expert + row0 * G);
            for (int off = 0; off < bytes; off += 1024)
              if (off + lane * 16 < bytes) dma16(s_src + off + lane * 16, dst + mat * bytes + off);
          }
        }
      }
    };
    const int64_t wave_rows = 16 * row_bytes;  // bytes between the A tiles of adjacent MMA waves
    const uint32_t lds_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_uchar_t*)(lds)));
    auto issue = [&](int g) {
      const int i = g / S;
      const int sj = g - i * S;
      if (i != cur) {
        setup_item(i);
        cur = i;
      }
      // LDS byte address of the step's buffer, kept wave-uniform (it goes to M0)
      const uint32_t buf = __builtin_amdgcn_readfirstlane(lds_base + static_cast<uint32_t>((g % D) * C::BUF));
      const int cb = c_begin + sj * KW;
#pragma unroll
      for (int k = 0; k < C::W_INSTR / NL; ++k) {
        // (MMA wave, A tile, slot) of this load; compile-time when one wave loads
        const int ii = k * NL + lw;
        const int u = ii % L;
        const int ai = (ii / L) % AT;
        const int cw = ii / (L * AT);
        const int c = min(cb + cw / WR, c_end - 1);
        dma16_to(wrow[ai][u] + ((cw % WR) * wave_rows + static_cast<int64_t>(c) * M::kChunkBytes), buf + ii * 1024);
      }
#pragma unroll
      for (int k = 0; k < XW; ++k) {
        const int c = min(cb + xkw[k], c_end - 1);
        dma16_to(xsrc[k] + static_cast<int64_t>(c) * CH * 2, buf + C::W_BYTES + (k * NL + lw) * 1024);
      }
    };
    // Loads complete in issue order, so "step s resident" = at most
    // (steps issued after s) * I_WAVE loads outstanding; an item's scale loads
    // are issued before its first step, so they only make the waits stricter.
    for (int g = 0; g < min(D - 1, total); ++g) issue(g);
    wait_vmcnt_steps<C::I_WAVE, D - 1>(min(D - 1, total) - 1);
    __builtin_amdgcn_s_barrier();  // step 0 resident
    for (int g = 0; g < total; ++g) {
      if (g + D - 1 < total) issue(g + D - 1);
      wait_vmcnt_steps<C::I_WAVE, D - 1>(max(0, min(total, g + D) - 1 - (g + 1)));
      if constexpr (KW > 1) {
        if (g % S == S - 1) __builtin_amdgcn_s_barrier();  // the MMA waves' partial-sum exchange
      }
      __builtin_amdgcn_s_barrier();  // step g consumed, step g+1 resident
    }
    return;
  }

  // ============================= MMA waves =============================
  const int q = lane >> 4;
  const int wr = wave % WR;
  const int kw = wave / WR;
  const int t16 = lane & 15;
  const bf16x8_t kOnes = __builtin_bit_cast(bf16x8_t, u32x4_t{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});

  f32x4_t acc[AT][NB];
#pragma unroll
  for (int ai = 0; ai < AT; ++ai)
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[ai][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  __syncthreads();  // step 0 resident

  for (int g = 0, i = 0, sj = 0; g < total; ++g) {
    const int c = c_begin + sj * KW + kw;
    if (c < c_end) {
      const unsigned char* buf = lds + (g % D) * C::BUF;
      uint4 wv[AT][L];
#pragma unroll
      for (int ai = 0; ai < AT; ++ai)
#pragma unroll
        for (int u = 0; u < L; ++u)
          wv[ai][u] = *reinterpret_cast<const uint4*>(buf + (wave * AT + ai) * L * 1024 + a_read_off<ENC>(lane, u));
      const unsigned char* xb = buf + C::W_BYTES + (kw * NTOK + t16) * C::ROWB;
      f32x4_t d[AT][NB];
      f32x4_t xs[NB];
      auto clear = [&]() {
#pragma unroll
        for (int ai = 0; ai < AT; ++ai)
#pragma unroll
          for (int b = 0; b < NB; ++b) d[ai][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int b = 0; b < NB; ++b) xs[b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      };
      auto kstep = [&](auto s_tag) {
        constexpr int S_ = decltype(s_tag)::value;
        const int slot = b_position(q, S_, t16, C::SPR);
        bf16x8_t bfr[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          bfr[b] = *reinterpret_cast<const bf16x8_t*>(xb + b * 16 * C::ROWB + slot * 16);
          // the chunk's activation sums on the matrix cores: a ones-matrix A
          // puts sum_k x[k][t] in every row of column t
          if constexpr (kScaled) xs[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kOnes, bfr[b], xs[b], 0, 0, 0);
        }
#pragma unroll
        for (int ai = 0; ai < AT; ++ai) {
          const bf16x8_t af = a_frag<ENC, S_>(wv[ai]);
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            if constexpr (kScaled)
              d[ai][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bfr[b], d[ai][b], 0, 0, 0);
            else
              acc[ai][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bfr[b], acc[ai][b], 0, 0, 0);
          }
        }
      };
      // one 128-element scale group h of the step: its four K-steps (sums
      // in d, xs), then acc += scale * (d - bias * sum(x))
      auto group = [&](auto h_tag) {
        constexpr int H_ = decltype(h_tag)::value;
        clear();
        kstep(std::integral_constant<int, 4 * H_>{});
        kstep(std::integral_constant<int, 4 * H_ + 1>{});
        kstep(std::integral_constant<int, 4 * H_ + 2>{});
        kstep(std::integral_constant<int, 4 * H_ + 3>{});
        float xsb[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) xsb[b] = M::kBias * xs[b][0];
        const int grp = (c * C::GPC + H_) / gdiv;
        const float* sc_item = scl + (i % SLOTS) * NMAT * WGR * G;
#pragma unroll
        for (int ai = 0; ai < AT; ++ai) {
          const int mat = NMAT == 2 ? ai : 0;
          const int rt = NMAT == 2 ? 0 : ai;
          const float* sr = sc_item + (mat * WGR + wr * 16 * RT + rt * 16 + 4 * q) * G + grp;
          const float s0 = sr[0], s1 = sr[G], s2 = sr[2 * G], s3 = sr[3 * G];
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            acc[ai][b][0] = fmaf(s0, d[ai][b][0] - xsb[b], acc[ai][b][0]);
            acc[ai][b][1] = fmaf(s1, d[ai][b][1] - xsb[b], acc[ai][b][1]);
            acc[ai][b][2] = fmaf(s2, d[ai][b][2] - xsb[b], acc[ai][b][2]);
            acc[ai][b][3] = fmaf(s3, d[ai][b][3] - xsb[b], acc[ai][b][3]);
          }
        }
      };
      if constexpr (kScaled) {
        group(std::integral_constant<int, 0>{});
        if constexpr (C::GPC > 1) group(std::integral_constant<int, 1>{});
      } else {
        kstep(std::integral_constant<int, 0>{});
        kstep(std::integral_constant<int, 1>{});
        if constexpr (KS > 2) {
          kstep(std::integral_constant<int, 2>{});
          kstep(std::integral_constant<int, 3>{});
        }
      }
    }
    if (sj == S - 1) {
      // ---- the item is complete: combine the K groups of waves, store ----
      bool writer = true;
      if constexpr (KW > 1) {
        constexpr int kVals = AT * NB * 4;
        if (kw > 0) {
#pragma unroll
          for (int ai = 0; ai < AT; ++ai)
#pragma unroll
            for (int b = 0; b < NB; ++b)
#pragma unroll
              for (int e = 0; e < 4; ++e)
                red[(((kw - 1) * WR + wr) * kVals + (ai * NB + b) * 4 + e) * 64 + lane] = acc[ai][b][e];
        }
        __syncthreads();
        writer = kw == 0;
        if (writer) {
#pragma unroll
          for (int o = 1; o < KW; ++o)
#pragma unroll
            for (int ai = 0; ai < AT; ++ai)
#pragma unroll
              for (int b = 0; b < NB; ++b)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                  acc[ai][b][e] += red[(((o - 1) * WR + wr) * kVals + (ai * NB + b) * 4 + e) * 64 + lane];
        }
      }
      if (writer) {
        const int* m = meta + i * META;
        const int nt = m[2];
        const int64_t row0 = static_cast<int64_t>(m[3]) * WGR;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const int tok = b * 16 + t16;
          if (tok >= nt) continue;
          const int route = m[4 + tok];
          if constexpr (MODE == kModeSilu) {
            const int64_t r0 = row0 + wr * 16 + 4 * q;
            uint16_t h[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) h[e] = f32_to_bf16(silu(round_bf16(acc[0][b][e])) * round_bf16(acc[1][b][e]));
            const uint2 v = make_uint2(static_cast<uint32_t>(h[0]) | (static_cast<uint32_t>(h[1]) << 16),
                                       static_cast<uint32_t>(h[2]) | (static_cast<uint32_t>(h[3]) << 16));
            *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(a.out) + static_cast<int64_t>(route) * a.ldo + r0) = v;
          } else {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
              const int64_t r0 = row0 + wr * 16 * RT + rt * 16 + 4 * q;
              float* dst = reinterpret_cast<float*>(a.out) + blockIdx.y * a.part_stride +
                           static_cast<int64_t>(route) * a.ldo + r0;
              *reinterpret_cast<float4*>(dst) =
                  make_float4(acc[rt][b][0], acc[rt][b][1], acc[rt][b][2], acc[rt][b][3]);
            }
          }
        }
      }
#pragma unroll
      for (int ai = 0; ai < AT; ++ai)
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[ai][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
    if (++sj == S) {
      sj = 0;
      ++i;
    }
    __syncthreads();  // step g consumed, step g+1 resident
  }
}

namespace {

template <int ENC, int NMAT, int MW, int NB, int KW>
size_t lds_bytes_for(int64_t K, int64_t group) {
  using C = MfmaCfg<ENC, NMAT, MW, NB, KW>;
  const size_t G = ENC == kBF16 ? 0 : static_cast<size_t>(K / group);
  return static_cast<size_t>(C::FIXED_LDS) + sizeof(float) * C::SLOTS * NMAT * G * C::WGR;
}

// The item's scale slot is rewritten SLOTS items later, when the loader issues
// that item's first step, up to D - 1 steps ahead of the MMA waves: safe when
// (SLOTS - 1) steps per item >= D - 1. And the ring, the slots and the
// metadata must fit the LDS.
template <int ENC, int NMAT, int MW, int NB, int KW>
bool cfg_fits(const MfmaArgs& a) {
  using C = MfmaCfg<ENC, NMAT, MW, NB, KW>;
  const int nch = static_cast<int>(a.K / C::CH);
  const int steps = (nch / (a.ksplit > 0 ? a.ksplit : 1)) / KW;
  if ((C::SLOTS - 1) * steps + 1 < C::D) return false;
  return lds_bytes_for<ENC, NMAT, MW, NB, KW>(a.K, a.group) <= 160 * 1024;
}

// Workgroups of one configuration that fit on a CU (cached per LDS size).
template <int ENC, int NMAT, int MW, int NB, int KW, int MODE>
int blocks_per_cu(size_t lds) {
  static std::atomic<int64_t> cache{-1};  // (lds << 8) | blocks
  const int64_t c = cache.load(std::memory_order_relaxed);
  if (c >= 0 && static_cast<size_t>(c >> 8) == lds) return static_cast<int>(c & 0xFF);
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, expert_mfma_kernel<ENC, NMAT, MW, NB, KW, MODE>,
                                                   MfmaCfg<ENC, NMAT, MW, NB, KW>::THREADS, lds) != hipSuccess ||
      n < 1)
    n = 1;
  if (n > 8) n = 8;
  cache.store((static_cast<int64_t>(lds) << 8) | n, std::memory_order_relaxed);
  return n;
}

template <int ENC, int NMAT, int MW, int NB, int KW>
hipError_t launch_cfg(const MfmaArgs& args, int cus, hipStream_t stream) {
  using C = MfmaCfg<ENC, NMAT, MW, NB, KW>;
  MfmaArgs a = args;
  a.row_blocks = static_cast<int32_t>(a.rows / C::WGR);
  if (!cfg_fits<ENC, NMAT, MW, NB, KW>(a)) return hipErrorInvalidValue;
  const size_t lds = lds_bytes_for<ENC, NMAT, MW, NB, KW>(a.K, a.group);
  constexpr int MODE = NMAT == 2 ? kModeSilu : kModeF32;
  auto kernel = expert_mfma_kernel<ENC, NMAT, MW, NB, KW, MODE>;
  if (lds > 64 * 1024) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess) return e;
  }
  // persistent grid: every resident slot once, more only if a run would exceed MAX_ITEMS
  const int64_t items = static_cast<int64_t>(a.row_blocks) * a.tile_bound;
  int64_t grid = static_cast<int64_t>(cus) * blocks_per_cu<ENC, NMAT, MW, NB, KW, MODE>(lds);
  const int64_t need = (items + C::MAX_ITEMS - 3) / (C::MAX_ITEMS - 2);
  if (grid < need) grid = need;
  if (grid > items) grid = items;
  grid = (grid + 7) & ~static_cast<int64_t>(7);
  hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(grid), static_cast<unsigned>(a.ksplit)), dim3(C::THREADS), lds,
                     stream, a);
  return hipGetLastError();
}

template <int ENC, int NMAT, int MW, int KW>
hipError_t launch_nb(const MfmaArgs& a, int nb, int cus, hipStream_t stream) {
  if (nb <= 1) return launch_cfg<ENC, NMAT, MW, 1, KW>(a, cus, stream);
  if constexpr (KW == 1) {
    if (nb <= 2) return launch_cfg<ENC, NMAT, MW, 2, KW>(a, cus, stream);
    if constexpr (MW == 8) {
      // 48-route tiles; the kernel's tile size must equal the tile list's
      if (nb == 3) return launch_cfg<ENC, NMAT, MW, 3, KW>(a, cus, stream);
    }
    if constexpr (MW == 4) {
      if (nb == 3) return hipErrorInvalidValue;
      if (nb <= 4) return launch_cfg<ENC, NMAT, MW, 4, KW>(a, cus, stream);
      // 128-route tiles exist for BF16 only (a smaller kernel tile would drop routes)
      if constexpr (ENC == kBF16) {
        if (nb <= 8) return launch_cfg<ENC, NMAT, MW, 8, KW>(a, cus, stream);
      }
    }
  }
  return hipErrorInvalidValue;
}

template <int ENC>
hipError_t launch_enc(int nmat, const MfmaArgs& a, int nb, int kw, int mw, int cus, hipStream_t stream) {
  if (nmat == 2) {
    if (kw == 4) return launch_nb<ENC, 2, 4, 4>(a, nb, cus, stream);
    if constexpr (ENC == kQ4) {  // Q8/BF16 gate+up tiles need too many registers for 8 MMA waves
      if (mw == 8) return launch_nb<ENC, 2, 8, 1>(a, nb, cus, stream);
    }
    return launch_nb<ENC, 2, 4, 1>(a, nb, cus, stream);
  }
  if (kw == 4) return launch_nb<ENC, 1, 4, 4>(a, nb, cus, stream);
  if (mw == 8) return launch_nb<ENC, 1, 8, 1>(a, nb, cus, stream);
  return launch_nb<ENC, 1, 4, 1>(a, nb, cus, stream);
}

// Q4 gate/up tiles of 16 routes on the wide form (K-steps of two scale
// groups, 8 rows x 128 B per weight load) when K is a multiple of 256 and the
// ring and scales fit the LDS (K up to ~2400 at 128-element groups). Returns
// hipErrorNotSupported when the call takes the narrow form. Measured against
// the narrow form and kept narrow: down tiles (c4 171.3 vs 167.0 us per call,
// c5 109.4 vs 97.9 with one workgroup per CU instead of two, batch 32 +1 us
// with K = 1408, whose odd group count left one step half used) and wider
// gate/up tiles (their rings do not fit).
hipError_t launch_q4_wide(int nmat, const MfmaArgs& a, int nb, int kw, int mw, int cus, hipStream_t stream) {
  if (nmat != 2 || nb != 1 || kw != 1 || a.group % 128 != 0 || a.K % 256 != 0) return hipErrorNotSupported;
  if (mw == 8) {
    if (!cfg_fits<kQ4Wide, 2, 8, 1, 1>(a)) return hipErrorNotSupported;
    return launch_cfg<kQ4Wide, 2, 8, 1, 1>(a, cus, stream);
  }
  if (!cfg_fits<kQ4Wide, 2, 4, 1, 1>(a)) return hipErrorNotSupported;
  return launch_cfg<kQ4Wide, 2, 4, 1, 1>(a, cus, stream);
}

}  // namespace

bool mfma_supported(int enc, int64_t rows, int64_t K, int64_t group) {
  if (rows <= 0 || rows % 64 != 0 || K < 768 || K % 128 != 0) return false;
  if (enc == kBF16) return true;
  return group > 0 && group % 128 == 0 && K % group == 0 && K / group <= 64;
}

hipError_t launch_expert_mfma(int enc, int nmat, const MfmaArgs& args, int nb, int kw, int mw, int cus,
                              hipStream_t stream) {
  MfmaArgs a = args;
  if (a.ksplit < 1) a.ksplit = 1;
  if (nmat == 2 && a.ksplit != 1) return hipErrorInvalidValue;
  if (kw != 1 && kw != 4) return hipErrorInvalidValue;
  if (mw != 4 && mw != 8) return hipErrorInvalidValue;
  if (kw == 4 && (nb > 1 || mw != 4)) return hipErrorInvalidValue;
  if (mw == 8 && nb > 3) return hipErrorInvalidValue;
  const int wgr = 16 * mw / kw;
  if (a.rows % wgr != 0) return hipErrorInvalidValue;
  if ((a.w_tail != nullptr || (a.rows_valid > 0 && a.rows_valid != a.rows)) && wgr != 16) return hipErrorInvalidValue;
  if (enc != kBF16) a.scales_per_expert = (a.rows * a.K + a.group - 1) / a.group;
  if (a.tile_bound <= 0) return hipSuccess;
  if (cus < 8) cus = 8;
  if (enc == kQ4) {
    const hipError_t e = launch_q4_wide(nmat, a, nb, kw, mw, cus, stream);
    if (e != hipErrorNotSupported) return e;
  }
  if (enc == kQ4) return launch_enc<kQ4>(nmat, a, nb, kw, mw, cus, stream);
  if (enc == kQ8) return launch_enc<kQ8>(nmat, a, nb, kw, mw, cus, stream);
  return launch_enc<kBF16>(nmat, a, nb, kw, mw, cus, stream);
}

}  // namespace uqm
