// Flash attention (forward) for 128-wide heads on gfx950 bf16 MFMA, with grouped K/V heads and
// the attention gate fused into the store; optionally with a per-batch key mask in which every
// query also keeps its own position (the text refiner's `mask | eye`).
//
// Workgroup = 4 waves sharing one K/V head: with G = heads / kv_heads query heads per K/V
// head, a workgroup serves hpw = min(G, 4) of them and 32 * QB * 4 / hpw query rows, one
// wave per (query head, 32*QB-row block). K/V tiles of KVT keys go global -> LDS by
// buffer_load_dwordx4 ... lds (no register staging) into a ring of STAGES buffers, and are
// read by all the workgroup's waves.
//
// Each wave computes S^T = K Q^T (v_mfma_f32_32x32x16_bf16, K fragments from LDS, Q
// fragments held in registers), so every lane owns one query column and half of the keys
// of the tile: the online-softmax row max / sum need a single cross-lane exchange (lane ^ 32).
// The probabilities, converted to bf16 in place, are exactly the B operand of O^T = V^T P^T
// (with a fixed permutation of the keys inside each 16-key step, applied identically to the
// V^T fragments), so P never leaves registers. V arrives transposed ([d, token]) with the
// middle two 4-key quads of every 16 keys swapped, so each V^T fragment is one 16-byte read.
//
// The softmax is VALU work beside the MFMAs, so it is kept short: exponentials are the bare
// v_exp_f32 of one fma (s * scale * log2(e) - max, a single rounding written out, so that every
// variant rounds alike; results below 2^-126 flush to zero, far under bf16 resolution of P),
// and the running output is rescaled only when the running max of some query column moved.
//
// LDS: K rows are 256 bytes, V^T rows 2*KVT bytes; chunk c of row r is stored at chunk
// c ^ swz(r) so the 16-lane phases of ds_read_b128 hit 64 distinct banks.
#include "iris_common.hpp"

#include <utility>

namespace iris {
namespace {

constexpr int kHd = 128;

struct AttnArgs {
  const bf16* q;
  const bf16* k;
  const bf16* vt;
  bf16* out0;
  bf16* out1;
  const bf16* gate0;
  const bf16* gate1;
  const unsigned char* key_mask;  // [batch, n_pad] 0/1 bytes, MASKED kernels only
  long ld_out, ld_gate;
  long out_brows0, out_brows1, gate_brows0, gate_brows1;
  int heads, kv_heads, n, n_pad, n_split;
  int hpw, rows_per_wg, n_qblocks, n_hgroups;
  int total_wg;
  float scale_log2;
};

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Chunk swizzle for LDS rows of CPR 16-byte chunks: rows of 256 bytes use c ^ (r % 16), of
// 128 bytes c ^ ((r / 2) % 8), of 64 bytes c ^ ((r / 4) % 4); 16 consecutive rows read at
// one logical chunk then cover all 64 banks.
template <int CPR>
__device__ __forceinline__ int swz(int r) {
  return (r / (16 / CPR)) % CPR;
}

// Store of one query row: lane owns query `row` and dims db*32 + 8 j + 4 g + (0..3) of head h;
// out = o / l, times sigmoid(gate) when a gate is given; rows past n_split go to out1.
__device__ __forceinline__ void store_row(const AttnArgs& p, const f32x16 (&o)[4], float l_lane, int b, int h, int row,
                                          int g) {
  const float l = l_lane + __shfl_xor(l_lane, 32);
  const float inv = 1.0f / l;
  if (row >= p.n) return;
  const bool first = row < p.n_split;
  bf16* out = first ? p.out0 : p.out1;
  const bf16* gate = first ? p.gate0 : p.gate1;
  const long r = first ? row : row - p.n_split;
  if (out == nullptr) return;
  bf16* orow_ptr = out + (b * (first ? p.out_brows0 : p.out_brows1) + r) * p.ld_out + h * kHd;
  const bf16* grow_ptr = gate ? gate + (b * (first ? p.gate_brows0 : p.gate_brows1) + r) * p.ld_gate + h * kHd : nullptr;
#pragma unroll
  for (int db = 0; db < 4; ++db) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int d0 = db * 32 + 8 * j + 4 * g;
      f32x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = o[db][4 * j + e] * inv;
      if (grow_ptr) {
        const f32x4 gv = load4(grow_ptr + d0);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] *= sigmoid(gv[e]);
      }
      store4(orow_ptr + d0, v);
    }
  }
}

// f(std::integral_constant<int, 0>{}), ..., f(std::integral_constant<int, N - 1>{}) in order.
template <int N, typename F, int... I>
__device__ __forceinline__ void unroll_stages_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void unroll_stages(F&& f) {
  unroll_stages_impl<N>(f, std::make_integer_sequence<int, N>{});
}

// STAGED: K/V tiles travel global -> registers (16-byte buffer loads) -> LDS (ds_write_b128)
// through two LDS stages: tile t + 1 is written while tile t is multiplied, tile t + 2 is
// loaded meanwhile. Otherwise a ring of STAGES tiles filled by buffer loads straight into LDS.
// MASKED: query q attends key j < n iff key_mask[b, j] != 0 or j == q. A tile can then hold no
// key of some query; its running max stays -inf and the exponentials use 0 in its place, so
// they are exactly 0 instead of NaN.
// NW: waves per workgroup; with NW = 12 (one workgroup per CU, three waves per SIMD: four query
// heads x three 32-row blocks) the first four waves fetch the K/V tiles that all twelve share,
// a third of the fetches of three 4-wave workgroups (ring only).
template <int QB, int STAGES, int KVT, bool STAGED, bool MASKED = false, int NW = 4>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(NW == 12 ? 3 : (QB == 1 ? 2 : 1)))) void
flash_attn_kernel(AttnArgs p) {  // 32-row waves: two or three waves per SIMD
  constexpr int KB = KVT / 32;     // 32-key blocks per tile
  constexpr int TILE = KVT * kHd;  // elements of one K (or V^T) tile
  constexpr int STAGE = 2 * TILE;  // K tile then V^T tile
  constexpr int LOADS = KVT / 16;  // 1 KB loads per fetching wave per operand per tile
  constexpr int LPW = 2 * LOADS;
  constexpr int VCPR = KVT / 8;    // 16-byte chunks per V^T row
  constexpr int VRPL = 64 / VCPR;  // V^T rows per 1 KB load
  static_assert(KVT == 32 || KVT == 64, "K/V tile of 32 or 64 keys");
  static_assert(STAGES >= 2 && (STAGES - 2) * LPW < 64 && (!STAGED || STAGES == 2), "pipeline depth");
  static_assert(NW == 4 || (NW == 12 && !STAGED), "twelve-wave workgroups use the LDS ring");
  __shared__ __attribute__((aligned(1024))) bf16 lds[STAGES * STAGE];

  // logical workgroup: (b, kv head, head group) major, query block minor; the XCD remap keeps
  // the query blocks of one K/V head on one XCD so its K/V stay in that L2.
  int wg = xcd_remap(blockIdx.x, p.total_wg);
  const int qblk = wg % p.n_qblocks;
  wg /= p.n_qblocks;
  const int hg = wg % p.n_hgroups;
  wg /= p.n_hgroups;
  const int kvh = wg % p.kv_heads;
  const int b = wg / p.kv_heads;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int l32 = lane & 31;
  const int g = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: LDS targets stay scalar
  const int group = p.heads / p.kv_heads;
  const int h = kvh * group + hg * p.hpw + (w % p.hpw);
  const int q0 = qblk * p.rows_per_wg + (w / p.hpw) * 32 * QB;
  const long n_pad = p.n_pad;

  // Q fragments: B operand of S^T = K Q^T; lane holds query q0 + qb*32 + l32, dims s*16 + g*8 .. +8
  const bf16* qh = p.q + (static_cast<long>(b) * p.heads + h) * n_pad * kHd;
  bf16x8 qf[QB][8];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const long row = min(static_cast<long>(q0 + qb * 32 + l32), n_pad - 1);
#pragma unroll
    for (int s = 0; s < 8; ++s) qf[qb][s] = *reinterpret_cast<const bf16x8*>(qh + row * kHd + s * 16 + g * 8);
  }

  const bf16* kh = p.k + (static_cast<long>(b) * p.kv_heads + kvh) * n_pad * kHd;
  const bf16* vh = p.vt + (static_cast<long>(b) * p.kv_heads + kvh) * kHd * n_pad;
  // per-lane fetch offsets: K load j of wave w covers key rows 4 (LOADS w + j) .. +4 (16 chunks
  // each), V^T load j covers dim rows VRPL (LOADS w + j) .. +VRPL (VCPR chunks each)
  int k_off[LOADS], v_off[LOADS];
#pragma unroll
  for (int j = 0; j < LOADS; ++j) {
    const int kr = (w * LOADS + j) * 4 + (lane >> 4);
    k_off[j] = kr * kHd + 8 * ((lane & 15) ^ swz<16>(kr));
    const int vd = (w * LOADS + j) * VRPL + lane / VCPR;
    v_off[j] = vd * static_cast<int>(n_pad) + 8 * ((lane % VCPR) ^ swz<VCPR>(vd));
  }
  // K and V^T of this (batch, K/V head) as buffer resources: a 32-bit VGPR byte offset per lane,
  // the tile position in an SGPR (n_pad < 2^23 keeps the offsets in range)
  const __amdgpu_buffer_rsrc_t rk =
      __builtin_amdgcn_make_buffer_rsrc((void*)kh, (short)0, static_cast<int>(n_pad) * kHd * 2, kBufferFlags);
  const __amdgpu_buffer_rsrc_t rv =
      __builtin_amdgcn_make_buffer_rsrc((void*)vh, (short)0, static_cast<int>(n_pad) * kHd * 2, kBufferFlags);
  // ring path: buffer loads straight into LDS. (global_load_lds with 64-bit VGPR addresses made
  // the compiler wait for every outstanding load, the ring's prefetch included, before the first
  // MFMA of each tile.)
  auto issue = [&](int t, int stage) {
    if (NW != 4 && w >= 4) return;  // (wave-uniform: the first four waves fetch)
    bf16* kl = lds + stage * STAGE;
    bf16* vl = kl + TILE;
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      buffer_load_lds16(rk, kl + (w * LOADS + j) * 512, k_off[j] * 2, t * KVT * kHd * 2);
      buffer_load_lds16(rv, vl + (w * LOADS + j) * 512, v_off[j] * 2, t * KVT * 2);
    }
  };
  // register-staged path: lane l's 16 bytes of load j land at byte 16 l of the same 1 KB blocks
  bf16x8 kreg[LOADS], vreg[LOADS];
  auto gload = [&](int t) {
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      kreg[j] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rk, k_off[j] * 2, t * KVT * kHd * 2, 0));
      vreg[j] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(rv, v_off[j] * 2, t * KVT * 2, 0));
    }
  };
  auto lwrite = [&](int stage) {
    bf16* kl = lds + stage * STAGE;
    bf16* vl = kl + TILE;
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      *reinterpret_cast<bf16x8*>(kl + (w * LOADS + j) * 512 + 8 * lane) = kreg[j];
      *reinterpret_cast<bf16x8*>(vl + (w * LOADS + j) * 512 + 8 * lane) = vreg[j];
    }
  };

  f32x16 o[4][QB];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) o[db][qb] = f32x16{};
  float m_run[QB], l_run[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) m_run[qb] = -INFINITY, l_run[qb] = 0.0f;
  const float sl2 = p.scale_log2;

  const int n_tiles = (p.n + KVT - 1) / KVT;
  if constexpr (STAGED) {
    gload(0);
    lwrite(0);
    gload(min(1, n_tiles - 1));
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): tile 0 written
    __builtin_amdgcn_s_barrier();
  } else {
#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s)
      if (s < n_tiles) issue(s, s);
  }
  // Tile t uses stage S = t % STAGES, a compile-time constant in each copy of the body (the loop
  // is unrolled by STAGES): the stage's LDS offsets become instruction immediates, so neither the
  // fragment addresses nor the ring's M0 bases cost per-tile VALU / SALU work.
  // Per-lane LDS byte offsets of the fragment reads, the same in every tile and stage (the
  // swizzle of a row depends on the lane's row within its 32-row block only): K step st of key
  // block kb at kb * 32 * 256 + k_rd[st] bytes, V^T (kb, jj) of dim block db at db * 32 * 2 KVT
  // + v_rd[kb][jj]. Each tile re-declares them opaque to the compiler (an empty asm), so the
  // stage and block constants fold into the reads' immediate offsets instead of becoming one
  // hoisted address register per stage.
  int k_rd[8], v_rd[KB][2];
#pragma unroll
  for (int st = 0; st < 8; ++st) k_rd[st] = 2 * (l32 * kHd + 8 * ((2 * st + g) ^ swz<16>(l32)));
#pragma unroll
  for (int kb = 0; kb < KB; ++kb)
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) v_rd[kb][jj] = 2 * (l32 * KVT + 8 * ((4 * kb + 2 * jj + g) ^ swz<VCPR>(l32)));

  auto tile = [&](const int t, auto stage) __attribute__((always_inline)) {
    constexpr int S = decltype(stage)::value;
#pragma unroll
    for (int st = 0; st < 8; ++st) asm volatile("" : "+v"(k_rd[st]));
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) asm volatile("" : "+v"(v_rd[kb][jj]));
    if constexpr (STAGED) {
      // tile t + 1 (loaded during tile t - 1) into the stage tile t - 1 used, then load tile
      // t + 2; past the end both repeat the last tile into a stage nothing reads again
      lwrite((S + 1) & 1);
      gload(min(t + 2, n_tiles - 1));
    } else {
      if (t + STAGES - 2 < n_tiles)
        wait_vmcnt<(STAGES - 2) * LPW>();
      else
        wait_vmcnt<0>();
      __builtin_amdgcn_s_barrier();  // tile t visible; stage (t-1) % STAGES no longer read
      if (t + STAGES - 1 < n_tiles) issue(t + STAGES - 1, (S + STAGES - 1) % STAGES);
    }
    const bf16* kl = lds + S * STAGE;
    const bf16* vl = kl + TILE;

    // S^T[key, q] for keys kb*32 + (8 (r/4) + 4 g + r%4), queries qb*32 + l32
    f32x16 s[KB][QB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) s[kb][qb] = f32x16{};
    // K fragments in a ring of KD k-steps: each MFMA's operand was requested KD - 1 MFMAs of
    // this wave earlier, so the LDS latency hides behind them
    constexpr int KD = KB == 1 ? 4 : 2;
    bf16x8 kf[KD][KB];
    auto read_k = [&](int st, int slot) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
        kf[slot][kb] = *reinterpret_cast<const bf16x8*>(reinterpret_cast<const char*>(kl + kb * 32 * kHd) + k_rd[st]);
    };
    // The S MFMAs issue at a raised wave priority: a wave in its MFMA phase is picked before the
    // waves of its SIMD that are in their softmax, which fill the gaps between its MFMAs
    // (trunk 4-5% and pixel-stage attention 8% faster than at one priority).
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(1);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int st = 0; st < KD; ++st) read_k(st, st);
#pragma unroll
    for (int st = 0; st < 8; ++st) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
          s[kb][qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[st % KD][kb], qf[qb][st], s[kb][qb], 0, 0, 0);
      if (st + KD < 8) read_k(st + KD, st % KD);
    }
    // keep that order (the scheduler would otherwise sink the reads to one MFMA ahead)
    __builtin_amdgcn_sched_group_barrier(0x100, KD * KB, 0);  // DS read
#pragma unroll
    for (int st = 0; st + KD < 8; ++st) {
      __builtin_amdgcn_sched_group_barrier(0x008, KB * QB, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, KB, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, KD * KB * QB, 0);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_sched_barrier(0);

    const int kv0 = t * KVT;
    if constexpr (MASKED) {
      // keys kv0 + kb*32 + 8 (r/4) + 4 g + r%4: four consecutive mask bytes per r/4
      const unsigned char* km = p.key_mask + static_cast<long>(b) * n_pad + kv0 + 4 * g;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const unsigned int bits = *reinterpret_cast<const unsigned int*>(km + kb * 32 + 8 * r4);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int key = kv0 + kb * 32 + 8 * r4 + 4 * g + e;
            const bool on = key < p.n && ((bits >> (8 * e)) & 0xffu) != 0;
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
              const bool keep = on || (key < p.n && key == q0 + qb * 32 + l32);
              if (!keep) s[kb][qb][4 * r4 + e] = -INFINITY;
            }
          }
        }
    } else if (kv0 + KVT > p.n) {  // tail tile: keys >= n do not exist (every tile holds at least one key)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kv0 + kb * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
          if (key >= p.n)
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) s[kb][qb][r] = -INFINITY;
        }
    }

    // Online softmax in the log2 domain, one query column per lane (and its partner lane ^ 32),
    // against the running max m_run, which is raised lazily: while every probability of the
    // tile stays <= 2^8 (each lane's partial sum <= 256) m_run and the output stay as they are;
    // otherwise (the first tile, a score more than 8 above m_run, a column with no key yet) the
    // columns that need it take their exact maxima, rescale their output and sums, and
    // recompute (the other columns keep their reference, so a column's result never depends on
    // its neighbours, padding rows included). The common path has no max reduction and no
    // output rescale. The sums add the FP32 exponentials in key order, one v_add_f32 each
    // (a v_dot2 of BF16 pairs beside the MFMAs costs several times more MFMA issue time).
    bf16x8 pf[KB][2][QB];
    auto probs = [&](int qb, float m) {
      float sum = 0.0f;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float x = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][qb][8 * jj + e], sl2, -m));
            pf[kb][jj][qb][e] = from_f32<bf16>(x);
            sum += x;
          }
      return sum;
    };
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      float sum = probs(qb, m_run[qb]);
      const int need = !(sum <= 256.0f);  // also for NaN / inf partial sums (the first tile)
      if (__any(need)) {                  // wave-uniform branch
        const int partner = __shfl_xor(need, 32);  // (every lane takes part in the exchange)
        const bool raise = need || partner;         // both halves of the column
        float mx = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][qb][r]);
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_max = fmaxf(m_run[qb], mx * sl2);
        const float m_new = !raise ? m_run[qb] : m_max;
        // A masked column with no key so far keeps max -inf (so that its first key, however low
        // its score, raises it: a finite stand-in would let every later probability underflow
        // to 0 and leave the row 0 / 0), and its all-masked tiles are evaluated against 0,
        // which gives exact zeros instead of NaN.
        const float m_ref = MASKED && m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m_run[qb] - m_ref);  // exactly 1 unless raised
        l_run[qb] *= alpha;
#pragma unroll
        for (int db = 0; db < 4; ++db) o[db][qb] *= alpha;
        m_run[qb] = m_new;
        sum = probs(qb, m_ref);
      }
      l_run[qb] += sum;
    }

    // O^T[d, q] += V^T[d, keys] P^T[keys, q], 16 keys per MFMA step: k-index g*8 + m is
    // key kb*32 + 16 jj + 8 (m / 4) + 4 g + m % 4 for both operands.
    // V^T fragments in a ring of VD steps, as the K fragments above
    constexpr int NV = KB * 2 * 4;  // (kb, jj, db) steps
    constexpr int VD = 4;
    bf16x8 vfr[VD];
    auto read_v = [&](int i, int slot) {
      const int kb = i / 8, jj = (i / 4) % 2, db = i % 4;
      vfr[slot] = *reinterpret_cast<const bf16x8*>(reinterpret_cast<const char*>(vl + db * 32 * KVT) + v_rd[kb][jj]);
    };
#pragma unroll
    for (int i = 0; i < VD; ++i) read_v(i, i);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int kb = i / 8, jj = (i / 4) % 2, db = i % 4;
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
        o[db][qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vfr[i % VD], pf[kb][jj][qb], o[db][qb], 0, 0, 0);
      if (i + VD < NV) read_v(i + VD, i % VD);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, VD, 0);
#pragma unroll
    for (int i = 0; i + VD < NV; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, QB, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, VD * QB, 0);
    if constexpr (STAGED) {
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): tile t + 1 written, tile t's reads done
      __builtin_amdgcn_s_barrier();
    }
  };
  int t0 = 0;
  for (; t0 + STAGES <= n_tiles; t0 += STAGES)
    unroll_stages<STAGES>([&](auto stage) {
      tile(t0 + decltype(stage)::value, stage);
      __builtin_amdgcn_sched_barrier(0);  // each tile's registers are dead before the next one
    });
  unroll_stages<STAGES - 1>([&](auto stage) {
    if (t0 + decltype(stage)::value < n_tiles) tile(t0 + decltype(stage)::value, stage);
  });
  if constexpr (STAGED) wait_vmcnt<0>();  // the repeated loads past the last tile

  // epilogue: lane owns query q0 + qb*32 + l32
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    f32x16 oq[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) oq[db] = o[db][qb];
    store_row(p, oq, l_run[qb], b, h, q0 + qb * 32 + l32, g);
  }
}

// Store of two 16-query blocks of a v_mfma_f32_16x16x32 O^T: o[db][qb][e] is dim 16 db + 4 h + e of
// query q0 + 16 qb + l16; the lane's partial row sum l_lane covers a quarter of the keys.
__device__ __forceinline__ void store_rows16(const AttnArgs& p, const f32x4 (&o)[8][2], const float (&l_lane)[2],
                                             int b, int hd, int q0, int l16, int h) {
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    float l = l_lane[qb] + __shfl_xor(l_lane[qb], 16);
    l += __shfl_xor(l, 32);
    const float inv = 1.0f / l;
    const int row = q0 + 16 * qb + l16;
    if (row >= p.n) continue;
    const bool first = row < p.n_split;
    bf16* out = first ? p.out0 : p.out1;
    const bf16* gate = first ? p.gate0 : p.gate1;
    const long r = first ? row : row - p.n_split;
    if (out == nullptr) continue;
    bf16* orow = out + (b * (first ? p.out_brows0 : p.out_brows1) + r) * p.ld_out + hd * kHd;
    const bf16* grow = gate ? gate + (b * (first ? p.gate_brows0 : p.gate_brows1) + r) * p.ld_gate + hd * kHd : nullptr;
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const int d0 = 16 * db + 4 * h;
      f32x4 v = o[db][qb] * inv;
      if (grow) {
        const f32x4 gv = load4(grow + d0);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] *= sigmoid(gv[e]);
      }
      store4(orow + d0, v);
    }
  }
}

// flash_attn_kernel's ring variants (twelve waves sharing a 3-stage ring of 32-key K / V^T tiles,
// or four waves with a 2-stage ring of 64-key tiles) on v_mfma_f32_16x16x32_bf16, which costs less
// power per FLOP than the 32 x 32 x 16 shape (the GPU is power-limited under MFMA load). A wave's
// 32 queries are two 16-query blocks; lane l (l16 = l % 16, h = l / 16) holds queries 16 qb + l16
// and, of each 32 keys of a tile, the keys kappa_kb(4 h + e) of key blocks kb = 0, 1 (e < 4), with
// kappa_0(r) = r + 8 (r / 8) and kappa_1(r) = kappa_0(r) + 8: the K fragment of block kb reads key
// rows kappa_kb(0..15), so that the lane's eight keys are exactly the eight V^T positions 8 h ..
// 8 h + 7 of those 32 keys in the V^T layout (the middle two 4-key quads of every 16 swapped) and
// P^T stays in registers as the B operand of O^T = V^T P^T. K rows are swizzled by swz_k (key % 16,
// bit 3 flipped for odd 16-key groups) so that the sixteen rows of one fragment read hit distinct
// banks. The softmax is the one of flash_attn_kernel (lazy max, FP32 sums in key order), over the
// four lanes of a query.
__device__ __forceinline__ int swz_k(int key) { return (key & 15) ^ (((key >> 4) & 1) << 3); }

template <int STAGES, int KVT, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(NW == 12 ? 3 : 2))) void
flash_attn16_kernel(AttnArgs p) {
  constexpr int H32 = KVT / 32;  // 32-key halves of a tile
  constexpr int NKB = 2 * H32;   // 16-key blocks
  constexpr int TILE = KVT * kHd, STAGE = 2 * TILE;
  constexpr int LOADS = KVT / 16, LPW = 2 * LOADS;
  constexpr int VCPR = KVT / 8, VRPL = 64 / VCPR;
  static_assert((KVT == 32 || KVT == 64) && (NW == 4 || NW == 12), "tile / workgroup shape");
  static_assert(STAGES >= 2 && (STAGES - 2) * LPW < 64, "pipeline depth");
  __shared__ __attribute__((aligned(1024))) bf16 lds[STAGES * STAGE];

  int wg = xcd_remap(blockIdx.x, p.total_wg);
  const int qblk = wg % p.n_qblocks;
  wg /= p.n_qblocks;
  const int hg = wg % p.n_hgroups;
  wg /= p.n_hgroups;
  const int kvh = wg % p.kv_heads;
  const int b = wg / p.kv_heads;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int l16 = lane & 15;
  const int h = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int group = p.heads / p.kv_heads;
  const int hd = kvh * group + hg * p.hpw + (w % p.hpw);
  const int q0 = qblk * p.rows_per_wg + (w / p.hpw) * 32;
  const long n_pad = p.n_pad;

  // Q fragments (B operand of S^T = K Q^T): query q0 + 16 qb + l16, dims 32 st + 8 h .. + 8
  const bf16* qh = p.q + (static_cast<long>(b) * p.heads + hd) * n_pad * kHd;
  bf16x8 qf[2][4];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const long row = min(static_cast<long>(q0 + 16 * qb + l16), n_pad - 1);
#pragma unroll
    for (int st = 0; st < 4; ++st) qf[qb][st] = *reinterpret_cast<const bf16x8*>(qh + row * kHd + 32 * st + 8 * h);
  }

  const bf16* kh = p.k + (static_cast<long>(b) * p.kv_heads + kvh) * n_pad * kHd;
  const bf16* vh = p.vt + (static_cast<long>(b) * p.kv_heads + kvh) * kHd * n_pad;
  // fetch offsets as flash_attn_kernel's, with the K rows swizzled by swz_k
  int k_off[LOADS], v_off[LOADS];
#pragma unroll
  for (int j = 0; j < LOADS; ++j) {
    const int kr = (w * LOADS + j) * 4 + (lane >> 4);
    k_off[j] = kr * kHd + 8 * ((lane & 15) ^ swz_k(kr));
    const int vd = (w * LOADS + j) * VRPL + lane / VCPR;
    v_off[j] = vd * static_cast<int>(n_pad) + 8 * ((lane % VCPR) ^ swz<VCPR>(vd));
  }
  const __amdgpu_buffer_rsrc_t rk =
      __builtin_amdgcn_make_buffer_rsrc((void*)kh, (short)0, static_cast<int>(n_pad) * kHd * 2, kBufferFlags);
  const __amdgpu_buffer_rsrc_t rv =
      __builtin_amdgcn_make_buffer_rsrc((void*)vh, (short)0, static_cast<int>(n_pad) * kHd * 2, kBufferFlags);
  auto issue = [&](int t, int stage) {
    if (NW != 4 && w >= 4) return;  // (wave-uniform: the first four waves fetch)
    bf16* kl = lds + stage * STAGE;
    bf16* vl = kl + TILE;
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      buffer_load_lds16(rk, kl + (w * LOADS + j) * 512, k_off[j] * 2, t * KVT * kHd * 2);
      buffer_load_lds16(rv, vl + (w * LOADS + j) * 512, v_off[j] * 2, t * KVT * 2);
    }
  };

  f32x4 o[8][2];
#pragma unroll
  for (int db = 0; db < 8; ++db) o[db][0] = o[db][1] = f32x4{};
  float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.0f, 0.0f};
  const float sl2 = p.scale_log2;

  const int n_tiles = (p.n + KVT - 1) / KVT;
#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < n_tiles) issue(s, s);
  // per-lane LDS byte offsets: K fragment (kb, st) at k_rd[kb][st] (key row 32 (kb / 2) +
  // kappa_{kb % 2}(l16), chunk 4 st + h), V^T fragment of dim block db and half hf at db * 16 * 2 KVT
  // + v_rd[hf] (dim row 16 db + l16, chunk 4 hf + h; a V^T row's swizzle does not depend on db)
  int k_rd[NKB][4], v_rd[H32];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) {
    const int key = 32 * (kb / 2) + l16 + 8 * (l16 >> 3) + 8 * (kb % 2);
#pragma unroll
    for (int st = 0; st < 4; ++st) k_rd[kb][st] = 2 * (key * kHd + 8 * ((4 * st + h) ^ swz_k(key)));
  }
#pragma unroll
  for (int hf = 0; hf < H32; ++hf) v_rd[hf] = 2 * (l16 * KVT + 8 * ((4 * hf + h) ^ swz<VCPR>(l16)));

  auto tile = [&](const int t, auto stage) __attribute__((always_inline)) {
    constexpr int S = decltype(stage)::value;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int st = 0; st < 4; ++st) asm volatile("" : "+v"(k_rd[kb][st]));
#pragma unroll
    for (int hf = 0; hf < H32; ++hf) asm volatile("" : "+v"(v_rd[hf]));
    if (t + STAGES - 2 < n_tiles)
      wait_vmcnt<(STAGES - 2) * LPW>();
    else
      wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();  // tile t visible; stage (t-1) % STAGES no longer read
    if (t + STAGES - 1 < n_tiles) issue(t + STAGES - 1, (S + STAGES - 1) % STAGES);
    const char* kl = reinterpret_cast<const char*>(lds + S * STAGE);
    const char* vl = reinterpret_cast<const char*>(lds + S * STAGE + TILE);

    // S^T[key, query 16 qb + l16] per 16-key block; K fragments (i = NKB st + kb) in a ring of 4
    constexpr int NK = 4 * NKB;
    f32x4 s[NKB][2];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) s[kb][0] = s[kb][1] = f32x4{};
    bf16x8 kf[4];
    auto read_k = [&](int i) { kf[i % 4] = *reinterpret_cast<const bf16x8*>(kl + k_rd[i % NKB][i / NKB]); };
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(1);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 4; ++i) read_k(i);
#pragma unroll
    for (int i = 0; i < NK; ++i) {
      const int st = i / NKB, kb = i % NKB;
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
        s[kb][qb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[i % 4], qf[qb][st], s[kb][qb], 0, 0, 0);
      if (i + 4 < NK) read_k(i + 4);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // DS read
#pragma unroll
    for (int i = 0; i + 4 < NK; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_sched_barrier(0);

    const int kv0 = t * KVT;
    if (kv0 + KVT > p.n) {  // tail tile: keys >= n do not exist
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * h + e;
          const int key = kv0 + 32 * (kb / 2) + r + 8 * (r >> 3) + 8 * (kb % 2);
          if (key >= p.n) s[kb][0][e] = s[kb][1][e] = -INFINITY;
        }
    }

    // online softmax as in flash_attn_kernel; a query's keys are spread over lanes l16 + 16 h
    bf16x8 pf[H32][2];
    auto probs = [&](int qb, float m) {
      float sum = 0.0f;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][qb][e], sl2, -m));
          pf[kb / 2][qb][4 * (kb % 2) + e] = from_f32<bf16>(x);
          sum += x;
        }
      return sum;
    };
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      float sum = probs(qb, m_run[qb]);
      const int need = !(sum <= 256.0f);  // also for NaN / inf partial sums (the first tile)
      if (__any(need)) {                  // wave-uniform branch
        int raise = need | __shfl_xor(need, 16);  // (every lane takes part in the exchanges)
        raise |= __shfl_xor(raise, 32);
        float mx = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int e = 0; e < 4; ++e) mx = fmaxf(mx, s[kb][qb][e]);
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = !raise ? m_run[qb] : fmaxf(m_run[qb], mx * sl2);
        const float alpha = __builtin_amdgcn_exp2f(m_run[qb] - m_new);  // exactly 1 unless raised
        l_run[qb] *= alpha;
#pragma unroll
        for (int db = 0; db < 8; ++db) o[db][qb] *= alpha;
        m_run[qb] = m_new;
        sum = probs(qb, m_new);
      }
      l_run[qb] += sum;
    }

    // O^T[dim 16 db + 4 h + e, query] += V^T[dims, keys] P^T[keys, query], one 32-key step per
    // half; V^T fragments (i = 8 hf + db) in a ring of 4
    constexpr int NV = 8 * H32;
    bf16x8 vfr[4];
    auto read_v = [&](int i) {
      vfr[i % 4] = *reinterpret_cast<const bf16x8*>(vl + (i % 8) * 16 * 2 * KVT + v_rd[i / 8]);
    };
#pragma unroll
    for (int i = 0; i < 4; ++i) read_v(i);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
        o[i % 8][qb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vfr[i % 4], pf[i / 8][qb], o[i % 8][qb], 0, 0, 0);
      if (i + 4 < NV) read_v(i + 4);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int i = 0; i + 4 < NV; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
  };
  int t0 = 0;
  for (; t0 + STAGES <= n_tiles; t0 += STAGES)
    unroll_stages<STAGES>([&](auto stage) {
      tile(t0 + decltype(stage)::value, stage);
      __builtin_amdgcn_sched_barrier(0);
    });
  unroll_stages<STAGES - 1>([&](auto stage) {
    if (t0 + decltype(stage)::value < n_tiles) tile(t0 + decltype(stage)::value, stage);
  });
  store_rows16(p, o, l_run, b, hd, q0, l16, h);
}

struct Variant {  // (the launch switch below picks the kernel of each)
  int qb, stages, kvt;
  bool staged;
  int nw = 4;
};
// 0: 32 query rows per wave, 64-key tiles staged through registers; 1: the same with 32-key
// tiles; 2: 64-key tiles, 2-stage ring; 3: 32-key tiles, 3-stage ring; 4: 32-key
// tiles in a 3-stage ring shared by twelve waves (four query heads x three row blocks); 5, 6:
// variants 4 and 2 on v_mfma_f32_16x16x32_bf16 (flash_attn16_kernel).
// (Measured and dropped: twelve-wave rings of 4 and 6 stages (1-2% slower than 3), eight of the
// twelve waves fetching instead of four (2% slower), 64-key tiles at twelve waves (spills); an
// eight-wave ping-pong of MFMA and softmax phases, 1.8x slower at the trunk shape; a
// software-pipelined wave issuing tile t - 1's P.V MFMAs around tile t's softmax, no faster than
// variant 1; a twelve-wave form issuing tile t + 1's S MFMAs between tile t's softmax
// instructions (4-stage ring), 1% faster than variant 4; 64- and 96-row waves at one wave per
// SIMD, 1.5-1.9x slower as compiled; the same 96-row, one-wave-per-SIMD form written as inline
// assembly (each MFMA carrying one score's exp / convert / add, P.V accumulators in fixed AGPRs,
// a 5- to 8-stage ring), bitwise equal to variant 1 and 4-6% slower than variant 4.)
constexpr Variant kVariants[] = {{1, 2, 64, true},  {1, 2, 32, true},      {1, 2, 64, false},    {1, 3, 32, false},
                                  {1, 3, 32, false, 12}, {1, 3, 32, false, 12}, {1, 2, 64, false}};
constexpr int kNumVariants = sizeof(kVariants) / sizeof(kVariants[0]);
// per thread: a forced variant never changes another thread's launches
thread_local int g_attn_variant = -1;

}  // namespace
}  // namespace iris

using namespace iris;

extern "C" int iris_flash_attn(const void* q, const void* k, const void* vt, int batch, int heads, int kv_heads,
                               long n, long n_pad, long n_split, float scale, void* out0, void* out1, long ld_out,
                               long out_batch_rows0, long out_batch_rows1, const void* gate0, const void* gate1,
                               long ld_gate, long gate_batch_rows0, long gate_batch_rows1, hipStream_t stream) {
  IRIS_REQUIRE(batch >= 0 && heads > 0 && kv_heads > 0 && heads % kv_heads == 0,
               "flash_attn: query heads %d must be a multiple of K/V heads %d", heads, kv_heads);
  const int group = heads / kv_heads;
  IRIS_REQUIRE((group & (group - 1)) == 0, "flash_attn: heads per K/V head must be a power of two (got %d)", group);
  IRIS_REQUIRE(n > 0 && n_pad >= n && n_pad % 64 == 0 && n_pad < (1L << 23),
               "flash_attn: n_pad must be n rounded up to a multiple of 64, below 2^23 (32-bit byte offsets)");
  IRIS_REQUIRE(n_split >= 0 && n_split <= n, "flash_attn: n_split outside [0, n]");
  IRIS_REQUIRE(ld_out >= heads * 128L && ld_out % 4 == 0, "flash_attn: bad ld_out");
  IRIS_REQUIRE((!gate0 && !gate1) || (ld_gate >= heads * 128L && ld_gate % 4 == 0), "flash_attn: bad ld_gate");
  IRIS_REQUIRE(out_batch_rows0 >= n_split && out_batch_rows1 >= n - n_split, "flash_attn: output batch stride too small");
  IRIS_REQUIRE((!gate0 || gate_batch_rows0 >= n_split) && (!gate1 || gate_batch_rows1 >= n - n_split),
               "flash_attn: gate batch stride too small");
  IRIS_REQUIRE(q && k && vt, "flash_attn: null input");
  IRIS_REQUIRE(aligned(q, 16) && aligned(k, 16) && aligned(vt, 16), "flash_attn: inputs must be 16-byte aligned");
  if (batch == 0) return IRIS_OK;
  AttnArgs args{};
  args.q = static_cast<const bf16*>(q);
  args.k = static_cast<const bf16*>(k);
  args.vt = static_cast<const bf16*>(vt);
  args.out0 = static_cast<bf16*>(out0);
  args.out1 = static_cast<bf16*>(out1);
  args.gate0 = static_cast<const bf16*>(gate0);
  args.gate1 = static_cast<const bf16*>(gate1);
  args.ld_out = ld_out;
  args.ld_gate = ld_gate;
  args.out_brows0 = out_batch_rows0;
  args.out_brows1 = out_batch_rows1;
  args.gate_brows0 = gate_batch_rows0;
  args.gate_brows1 = gate_batch_rows1;
  args.heads = heads;
  args.kv_heads = kv_heads;
  args.n = static_cast<int>(n);
  args.n_pad = static_cast<int>(n_pad);
  args.n_split = static_cast<int>(n_split);
  args.hpw = group < 4 ? group : 4;
  // Grouped heads (the trunk's 20 query / 5 K/V heads): twelve-wave workgroups sharing one K/V
  // ring (one per CU; 230 of them cover a 4352-token sequence) on the 16 x 16 x 32 MFMA when
  // their rounds over the CUs are at least 80% full (variant 5; the 32 x 32 x 16 form, variant 4,
  // was 9-11% faster than variant 1 there, and variant 5 took the step 0.15-0.2 ms below variant
  // 4); else 32-key tiles staged through registers in three 4-wave workgroups per CU (variant 1:
  // 168 VGPRs; small grids spread over more CUs). One query head per K/V head (the pixel stage):
  // 64-key tiles in a 2-stage ring. Each measured fastest at its shapes.
  // The choice depends on one batch item's shape only: variant 5 rounds differently from
  // variant 1, and a row's result must not depend on the other items of its batch.
  int variant = g_attn_variant;
  if (variant < 0) {
    variant = group >= 4 ? 1 : 2;
    if (group >= 4) {
      const int cus = device_cus();
      const long wide = static_cast<long>(kv_heads) * (group / 4) * ((n + 95) / 96);
      const long rounds = (wide + cus - 1) / cus;
      if (wide >= 0.8 * rounds * cus) variant = 5;
    }
  }
  const Variant v = kVariants[variant];
  args.rows_per_wg = 32 * v.qb * v.nw / args.hpw;
  args.n_qblocks = static_cast<int>((n + args.rows_per_wg - 1) / args.rows_per_wg);
  args.n_hgroups = group / args.hpw;
  const long total = static_cast<long>(batch) * kv_heads * args.n_hgroups * args.n_qblocks;
  IRIS_REQUIRE(total < (1L << 31), "flash_attn: grid too large");
  args.total_wg = static_cast<int>(total);
  args.scale_log2 = scale * 1.4426950408889634f;
  const dim3 grid(args.total_wg);
  switch (variant) {
    case 0:
      flash_attn_kernel<1, 2, 64, true><<<grid, 256, 0, stream>>>(args);
      break;
    case 1:
      flash_attn_kernel<1, 2, 32, true><<<grid, 256, 0, stream>>>(args);
      break;
    case 2:
      flash_attn_kernel<1, 2, 64, false><<<grid, 256, 0, stream>>>(args);
      break;
    case 3:
      flash_attn_kernel<1, 3, 32, false><<<grid, 256, 0, stream>>>(args);
      break;
    case 4:
      flash_attn_kernel<1, 3, 32, false, false, 12><<<grid, dim3(768), 0, stream>>>(args);
      break;
    case 5:
      flash_attn16_kernel<3, 32, 12><<<grid, dim3(768), 0, stream>>>(args);
      break;
    default:
      flash_attn16_kernel<2, 64, 4><<<grid, 256, 0, stream>>>(args);
      break;
  }
  return check_launch("flash_attn");
}

extern "C" int iris_flash_attn_masked(const void* q, const void* k, const void* vt, int batch, int heads,
                                      int kv_heads, long n, long n_pad, float scale, const void* key_mask,
                                      void* out, long ld_out, long out_batch_rows, hipStream_t stream) {
  IRIS_REQUIRE(batch >= 0 && heads > 0 && kv_heads > 0 && heads % kv_heads == 0,
               "flash_attn_masked: query heads %d must be a multiple of K/V heads %d", heads, kv_heads);
  const int group = heads / kv_heads;
  IRIS_REQUIRE((group & (group - 1)) == 0, "flash_attn_masked: heads per K/V head must be a power of two (got %d)",
               group);
  IRIS_REQUIRE(n > 0 && n_pad >= n && n_pad % 64 == 0 && n_pad < (1L << 23),
               "flash_attn_masked: n_pad must be n rounded up to a multiple of 64, below 2^23 (32-bit byte offsets)");
  IRIS_REQUIRE(ld_out >= heads * 128L && ld_out % 4 == 0 && out_batch_rows >= n, "flash_attn_masked: bad output strides");
  IRIS_REQUIRE(q && k && vt && key_mask && out, "flash_attn_masked: null pointer");
  IRIS_REQUIRE(aligned(q, 16) && aligned(k, 16) && aligned(vt, 16) && aligned(key_mask, 4) && aligned(out, 8),
               "flash_attn_masked: misaligned pointer");
  if (batch == 0) return IRIS_OK;
  AttnArgs args{};
  args.q = static_cast<const bf16*>(q);
  args.k = static_cast<const bf16*>(k);
  args.vt = static_cast<const bf16*>(vt);
  args.out1 = static_cast<bf16*>(out);
  args.key_mask = static_cast<const unsigned char*>(key_mask);
  args.ld_out = ld_out;
  args.out_brows1 = out_batch_rows;
  args.heads = heads;
  args.kv_heads = kv_heads;
  args.n = static_cast<int>(n);
  args.n_pad = static_cast<int>(n_pad);
  args.n_split = 0;
  args.hpw = group < 4 ? group : 4;
  args.rows_per_wg = 32 * 4 / args.hpw;
  args.n_qblocks = static_cast<int>((n + args.rows_per_wg - 1) / args.rows_per_wg);
  args.n_hgroups = group / args.hpw;
  const long total = static_cast<long>(batch) * kv_heads * args.n_hgroups * args.n_qblocks;
  IRIS_REQUIRE(total < (1L << 31), "flash_attn_masked: grid too large");
  args.total_wg = static_cast<int>(total);
  args.scale_log2 = scale * 1.4426950408889634f;
  // 32-key tiles: the mask logic fits in the registers of two workgroups per CU
  flash_attn_kernel<1, 2, 32, true, true><<<dim3(args.total_wg), 256, 0, stream>>>(args);
  return check_launch("flash_attn_masked");
}

// Tuning hook: force an attention variant (an index into kVariants) or restore the automatic
// choice (-1).
extern "C" int iris_flash_attn_force_variant(int variant) {
  IRIS_REQUIRE(variant >= -1 && variant < kNumVariants, "flash_attn_force_variant: variant in -1..%d",
               kNumVariants - 1);
  g_attn_variant = variant;
  return IRIS_OK;
}
