// Dense BF16 GEMM on the MFMA cores: the shared expert of calls with many
// tokens (prefill).
//
// Serves, for those calls, the shared expert's three dense linears in the
// reference's Qwen block (src/uma_qmoe/qwen_compressed_loader.py:72, the
// Transformers Qwen2MoeMLP: down(silu(gate(x)) * up(x)) over bf16 weights). The
// expert-grouped kernel (uqm_mfma.hip) gives every MMA wave one 16-row strip of
// weights and the whole route tile, which suits routed experts with few routes
// each; on a dense matrix at hundreds of tokens it makes every wave re-read the
// whole activation tile from LDS, and its waves read a step's fragments and
// then run its MFMAs in lock step. Here the output tile is square:
//   * a workgroup of 4 or 8 waves computes 128 weight rows x 128 or 256
//     tokens, each wave a 64 x 64 block: 4 row tiles x 4 token tiles of
//     v_mfma_f32_16x16x32_bf16 (64 FP32 accumulators per lane). Gate/up items
//     take rows r .. r+63 of both matrices and give each wave the same 32 rows
//     of gate and of up, so the SiLU epilogue pairs them in registers;
//   * K advances 64 elements per stage; every wave issues a quarter of each
//     stage's loads (global_load_lds, 16 bytes per lane, no registers) into a
//     ring of 4 stages of 32 KB or 3 of 48 KB, all but one ahead of the stage
//     being computed;
//   * each 32-element chunk's fragments are read from LDS while the previous
//     chunk's MFMAs run (two register sets); the barrier of a stage only hands
//     a ring buffer back to the loads;
//   * a staged row is 128 bytes; its 16-byte slot p sits at position
//     p ^ ((row >> 1) & 7), so the 16 rows of a fragment read (128 bytes apart)
//     fall on 16 distinct groups of 4 banks.
// Work items (row block x token tile x K split) are dealt to the eight XCDs
// in contiguous ranges, the token tiles of one row block next to each other, so
// the workgroups that share a row block run together on one XCD and read its
// rows from HBM once.
//
// MFMA operand layout (as in uqm_mfma.hip): A lane l holds row l%16 and
// K-slice 8*(l/16)..+7; B lane l holds token l%16, same K-slice; D lane l holds
// token l%16, rows 4*(l/16)+i.
#include "uqm_dense.h"

#include "uqm_internal.h"

namespace uqm {
namespace {

typedef __attribute__((address_space(3))) void dense_lds_t;

constexpr int kStepK = 64;             // K elements per stage
constexpr int kRowBytes = 2 * kStepK;  // one staged row
constexpr int kRegionA = 128 * kRowBytes;  // 128 weight rows

// WAVES = 4: 128-token items, a ring of 4 stages of 32 KB (one wave per SIMD);
// WAVES = 8: 256-token items, 3 stages of 48 KB (two waves per SIMD: twice the
// MFMA work per stage barrier, and one wave's MFMAs run while the other waits).
template <int WAVES>
struct DenseCfg {
  static_assert(WAVES == 4 || WAVES == 8, "4 or 8 waves");
  static constexpr int kTokens = 32 * WAVES;                // tokens per work item
  static constexpr int kRegionB = kTokens * kRowBytes;      // the item's tokens
  static constexpr int kStageBytes = kRegionA + kRegionB;
  static constexpr int kStages = WAVES == 8 ? 3 : 4;
  static constexpr int kLoadsA = kRegionA / 1024 / WAVES;  // 1 KB loads per wave and stage
  static constexpr int kLoadsB = kRegionB / 1024 / WAVES;
  static constexpr int kLoadsPerWave = kLoadsA + kLoadsB;
  static constexpr size_t kLds = static_cast<size_t>(kStages) * kStageBytes;
  static constexpr int kThreads = 64 * WAVES;
  static_assert(kLds <= 144 * 1024, "LDS ring too large");
  static_assert((kStages - 1) * kLoadsPerWave <= 63, "outstanding loads must fit vmcnt");
};

template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N <= 63, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Waits until at most n stages (PER loads each) of this wave's loads are
// outstanding (loads complete in issue order; 0 <= n <= 3, wave-uniform).
template <int PER>
__device__ __forceinline__ void wait_stages(int n) {
  if (n >= 3)
    wait_vm<3 * PER>();
  else if (n == 2)
    wait_vm<2 * PER>();
  else if (n == 1)
    wait_vm<PER>();
  else
    wait_vm<0>();
}

// This wave's LDS reads complete, then the workgroup barrier. (Its loads into
// LDS are waited for separately, by stage; a plain __syncthreads would wait for
// all of them.)
__device__ __forceinline__ void stage_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), vmcnt and expcnt unlimited
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

// This wave's LDS reads complete. (Waited for before the next chunk's reads
// are issued, a chunk after their own issue, so the MFMAs that follow need no
// wait: left to itself the compiler waits for every read in flight, the ones
// just issued included, before the first MFMA.)
__device__ __forceinline__ void reads_done() {
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_sched_barrier(0);
}

// 16 bytes per lane from global memory into LDS at a wave-uniform LDS byte
// address (lane l's bytes at lds_addr + 16 l). (A helper of its own: with the
// builtin written in the kernel body the host compilation drops the kernels'
// launch stubs.)
__device__ __forceinline__ void dma16_to(const void* src, uint32_t lds_addr) {
  __builtin_amdgcn_global_load_lds(src, reinterpret_cast<dense_lds_t*>(static_cast<uintptr_t>(lds_addr)), 16, 0, 0);
}

// Byte offset of 16-byte slot `slot` of staged row `row`.
__device__ __forceinline__ uint32_t slot_at(int row, int slot) {
  return static_cast<uint32_t>(row * kRowBytes + ((slot ^ ((row >> 1) & 7)) << 4));
}

}  // namespace

// (At least two waves per SIMD for the register budget: at most 256 VGPRs, so
// the accumulators stay in VGPRs with each MFMA's result in its own input
// registers; with 512 the compiler moves them through AGPRs around every MFMA.
// One workgroup per CU runs, bound by its LDS ring.)
template <int MODE, int WAVES>
__global__ __launch_bounds__(64 * WAVES, 2) void dense_mfma_kernel(DenseArgs a) {
  using C = DenseCfg<WAVES>;
  constexpr int kTokens = C::kTokens, kStages = C::kStages, kStageBytes = C::kStageBytes;
  constexpr int kLoadsA = C::kLoadsA, kLoadsB = C::kLoadsB;
  constexpr bool kSilu = MODE == kModeSilu;
  constexpr int RB = kSilu ? 64 : 128;  // rows per item per matrix
  extern __shared__ __align__(16) unsigned char lds[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int wr = wave & 1, wt = wave >> 1;
  const int r16 = lane & 15, q = lane >> 4;

  // ---- this workgroup's items ----
  const int nN = static_cast<int>((a.rows + RB - 1) / RB);
  const int nT = static_cast<int>((a.T + kTokens - 1) / kTokens);
  const int NI = nN * a.ksplit * nT;
  const int xcd = static_cast<int>(blockIdx.x & 7u);
  const int per = static_cast<int>(gridDim.x >> 3);
  const int wslot = static_cast<int>(blockIdx.x >> 3);
  const int xb = static_cast<int>(static_cast<int64_t>(NI) * xcd / 8);
  const int xe = static_cast<int>(static_cast<int64_t>(NI) * (xcd + 1) / 8);
  const int nit = xe - xb - wslot > 0 ? (xe - xb - wslot + per - 1) / per : 0;
  if (nit == 0) return;  // uniform over the workgroup
  const int S = static_cast<int>(a.K / kStepK) / a.ksplit;  // stages per item
  const int total = nit * S;
  struct Item {
    int rb, tb, split;
  };
  auto item_of = [&](int i) {
    const int it = xb + wslot + i * per;
    const int grp = it / nT;
    Item r;
    r.tb = it - grp * nT;
    r.split = grp / nN;
    r.rb = grp - r.split * nN;
    return r;
  };

  const uint32_t lds_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((dense_lds_t*)(lds)));

  // ---- loads: this wave's 4 weight and 4 activation loads of stage g ----
  // Load d (0..15) of a region covers staged rows 8d .. 8d+7; lane l fills
  // position l%8 of row 8d + l/8 with slot (l%8) ^ ((row >> 1) & 7). The lane's
  // source rows are set up once per item (clamped to the last row / token).
  // (kernel arguments read once: a scalar load in flight inside the loop would
  // make every LDS wait there a full one)
  const uint16_t* const wsel = kSilu && wave >= WAVES / 2 ? a.w[1] : a.w[0];  // weight loads 8-15: up rows
  const uint16_t* const xbase = a.x;
  const int64_t rows = a.rows, K = a.K, T = a.T, ldx = a.ldx, ldo = a.ldo, part_stride = a.part_stride;
  void* const out = a.out;
  const uint16_t* wsrc[kLoadsA];
  const uint16_t* xsrc[kLoadsB];
  int issued_item = -1, issue_split = 0;
  auto setup_loads = [&](int i) {
    const Item it = item_of(i);
    issue_split = it.split;
#pragma unroll
    for (int u = 0; u < kLoadsA; ++u) {
      const int row = 8 * (kLoadsA * wave + u) + (lane >> 3);
      const int slot = (lane & 7) ^ ((row >> 1) & 7);
      int64_t wrow = static_cast<int64_t>(it.rb) * RB + (kSilu ? (row & 63) : row);
      if (wrow >= rows) wrow = rows - 1;
      wsrc[u] = wsel + wrow * K + 8 * slot;
    }
#pragma unroll
    for (int u = 0; u < kLoadsB; ++u) {
      const int row = 8 * (kLoadsB * wave + u) + (lane >> 3);
      const int slot = (lane & 7) ^ ((row >> 1) & 7);
      int64_t t = static_cast<int64_t>(it.tb) * kTokens + row;
      if (t >= T) t = T - 1;
      xsrc[u] = xbase + t * ldx + 8 * slot;
    }
  };
  auto issue = [&](int g) {
    const int i = g / S;
    if (i != issued_item) {
      setup_loads(i);
      issued_item = i;
    }
    const int64_t k0 = static_cast<int64_t>(issue_split * S + (g - i * S)) * kStepK;
    const uint32_t buf = __builtin_amdgcn_readfirstlane(lds_base + static_cast<uint32_t>((g % kStages) * kStageBytes));
#pragma unroll
    for (int u = 0; u < kLoadsA; ++u) dma16_to(wsrc[u] + k0, buf + (kLoadsA * wave + u) * 1024);
#pragma unroll
    for (int u = 0; u < kLoadsB; ++u) dma16_to(xsrc[u] + k0, buf + kRegionA + (kLoadsB * wave + u) * 1024);
  };

  // ---- fragments of one 32-element chunk ----
  struct Frags {
    bf16x8_t fa[4];
    bf16x8_t fb[4];
  };
  // staged row of this lane in A tile mt (its base is a multiple of 16, so the
  // slot swizzle depends on r16 only)
  auto a_base = [&](int mt) { return kSilu ? 64 * (mt >> 1) + 32 * wr + 16 * (mt & 1) : 64 * wr + 16 * mt; };
  const uint32_t off0 = slot_at(r16, q), off1 = slot_at(r16, 4 + q);
  auto read = [&](int g, int c, Frags& f) {
    const unsigned char* buf = lds + (g % kStages) * kStageBytes + (c ? off1 : off0);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) f.fa[mt] = *reinterpret_cast<const bf16x8_t*>(buf + a_base(mt) * kRowBytes);
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
      f.fb[tt] = *reinterpret_cast<const bf16x8_t*>(buf + kRegionA + (64 * wt + 16 * tt) * kRowBytes);
  };

  f32x4_t acc[4][4];
  auto mfma = [&](const Frags& f) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
        acc[mt][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.fa[mt], f.fb[tt], acc[mt][tt], 0, 0, 0);
  };

  auto store = [&](int i) {
    const Item it = item_of(i);
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const int64_t t = static_cast<int64_t>(it.tb) * kTokens + 64 * wt + 16 * tt + r16;
      if (t >= T) continue;
      if constexpr (kSilu) {
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
          const int64_t n = static_cast<int64_t>(it.rb) * RB + 32 * wr + 16 * rt + 4 * q;
          if (n >= rows) continue;
          uint16_t h[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) h[e] = f32_to_bf16(silu(round_bf16(acc[rt][tt][e])) * round_bf16(acc[2 + rt][tt][e]));
          const uint2 v = make_uint2(static_cast<uint32_t>(h[0]) | (static_cast<uint32_t>(h[1]) << 16),
                                     static_cast<uint32_t>(h[2]) | (static_cast<uint32_t>(h[3]) << 16));
          *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + t * ldo + n) = v;
        }
      } else {
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          const int64_t n = static_cast<int64_t>(it.rb) * RB + 64 * wr + 16 * mt + 4 * q;
          if (n >= rows) continue;
          float* dst = static_cast<float*>(out) + it.split * part_stride + t * ldo + n;
          *reinterpret_cast<float4*>(dst) = make_float4(acc[mt][tt][0], acc[mt][tt][1], acc[mt][tt][2], acc[mt][tt][3]);
        }
      }
    }
  };

  // Stage g: chunk 1 is read while chunk 0's MFMAs run; then the wait for
  // stage g+1's loads and the barrier that hands buffer g back to the loads
  // (stage g+4 goes there), and chunk 0 of stage g+1 is read while chunk 1's
  // MFMAs run.
  const int pro = min(total, kStages);
  for (int g = 0; g < pro; ++g) issue(g);
  wait_stages<C::kLoadsPerWave>(pro - 1);
  stage_barrier();
  Frags f0, f1;
  read(0, 0, f0);
  for (int i = 0, g = 0; i < nit; ++i) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) acc[mt][tt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < S; ++j, ++g) {
      reads_done();
      read(g, 1, f1);
      mfma(f0);
      // (also after the last stage, where the read finds a stale buffer: a
      // branch around it would make the compiler wait for it before the MFMAs)
      wait_stages<C::kLoadsPerWave>(max(0, min(total - g - 2, kStages - 2)));
      stage_barrier();  // f1's reads done too
      if (g + kStages < total) issue(g + kStages);
      read(g + 1, 0, f0);
      mfma(f1);
    }
    store(i);
  }
}

bool dense_supported(int64_t rows, int64_t K, int64_t T) {
  return rows > 0 && rows % 64 == 0 && K >= 256 && K % kStepK == 0 && T >= kDenseMinTokens;
}

namespace {

int64_t dense_items(int nmat, int64_t rows, int64_t T, int waves, int ksplit) {
  const int64_t rb = nmat == 2 ? 64 : 128;
  const int64_t tok = 32 * waves;
  return (rows + rb - 1) / rb * ksplit * ((T + tok - 1) / tok);
}

template <int MODE, int WAVES>
hipError_t launch_cfg(const DenseArgs& a, int cus, hipStream_t stream) {
  using C = DenseCfg<WAVES>;
  const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&dense_mfma_kernel<MODE, WAVES>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(C::kLds));
  if (e != hipSuccess) return e;
  // persistent grid: one workgroup per CU (the ring takes 128-144 KB of LDS),
  // a multiple of 8 so that every XCD gets the same number
  const int64_t items = dense_items(MODE == kModeSilu ? 2 : 1, a.rows, a.T, WAVES, a.ksplit);
  int64_t grid = cus < items ? cus : items;
  grid = (grid + 7) & ~static_cast<int64_t>(7);
  if (grid < 8) grid = 8;
  hipLaunchKernelGGL((dense_mfma_kernel<MODE, WAVES>), dim3(static_cast<unsigned>(grid)), dim3(C::kThreads), C::kLds,
                     stream, a);
  return hipGetLastError();
}

}  // namespace

DensePlan plan_dense(int nmat, int64_t rows, int64_t K, int64_t T, int cus, int max_split) {
  // Relative time of one stage: the 8-wave item (128 x 256) takes ~1.4 times
  // as long per stage as the 4-wave one (128 x 128) for twice the work
  // (c4 gate/up: 1.1 vs 0.79 us per stage).
  const int64_t steps = K / kStepK;
  const int64_t grid = cus < 8 ? 8 : cus;
  DensePlan best{4, 1};
  double best_cost = -1.0;
  for (int waves = 4; waves <= 8; waves *= 2) {
    for (int ks = 1; ks <= (nmat == 2 ? 1 : max_split); ks *= 2) {
      if (steps % ks != 0) continue;
      const int64_t rounds = (dense_items(nmat, rows, T, waves, ks) + grid - 1) / grid;
      const double cost = static_cast<double>(rounds * (steps / ks)) * (waves == 8 ? 1.4 : 1.0);
      if (best_cost < 0.0 || cost < best_cost) {  // ties: fewer waves, smaller split
        best_cost = cost;
        best = DensePlan{waves, ks};
      }
    }
  }
  return best;
}

hipError_t launch_dense_mfma(int nmat, const DenseArgs& args, int waves, int cus, hipStream_t stream) {
  DenseArgs a = args;
  if (nmat != 1 && nmat != 2) return hipErrorInvalidValue;
  if (waves != 4 && waves != 8) return hipErrorInvalidValue;
  if (!dense_supported(a.rows, a.K, a.T)) return hipErrorInvalidValue;
  if (a.ksplit < 1) a.ksplit = 1;
  if (nmat == 2 && a.ksplit != 1) return hipErrorInvalidValue;
  if ((a.K / kStepK) % a.ksplit != 0) return hipErrorInvalidValue;
  if (nmat == 2) return waves == 8 ? launch_cfg<kModeSilu, 8>(a, cus, stream) : launch_cfg<kModeSilu, 4>(a, cus, stream);
  return waves == 8 ? launch_cfg<kModeF32, 8>(a, cus, stream) : launch_cfg<kModeF32, 4>(a, cus, stream);
}

}  // namespace uqm
