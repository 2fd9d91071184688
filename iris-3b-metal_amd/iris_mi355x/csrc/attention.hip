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
  for (int t = 0; t < n_tiles; ++t) {
    if constexpr (STAGED) {
      // tile t + 1 (loaded during tile t - 1) into the stage tile t - 1 used, then load tile
      // t + 2; past the end both repeat the last tile into a stage nothing reads again
      lwrite((t + 1) & 1);
      gload(min(t + 2, n_tiles - 1));
    } else {
      if (t + STAGES - 2 < n_tiles)
        wait_vmcnt<(STAGES - 2) * LPW>();
      else
        wait_vmcnt<0>();
      __builtin_amdgcn_s_barrier();  // tile t visible; stage (t-1) % STAGES no longer read
      if (t + STAGES - 1 < n_tiles) issue(t + STAGES - 1, (t + STAGES - 1) % STAGES);
    }
    const bf16* kl = lds + (t % STAGES) * STAGE;
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
      for (int kb = 0; kb < KB; ++kb) {
        const int r = kb * 32 + l32;
        kf[slot][kb] = *reinterpret_cast<const bf16x8*>(kl + r * kHd + 8 * ((2 * st + g) ^ swz<16>(r)));
      }
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
        // (a column with no key so far takes a finite reference, so masked tiles give 0, not NaN)
        const float m_new = !raise ? m_run[qb] : (MASKED && m_max == -INFINITY ? 0.0f : m_max);
        const float alpha = __builtin_amdgcn_exp2f(m_run[qb] - m_new);  // exactly 1 unless raised
        l_run[qb] *= alpha;
#pragma unroll
        for (int db = 0; db < 4; ++db) o[db][qb] *= alpha;
        m_run[qb] = m_new;
        sum = probs(qb, m_new);
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
      const int c = 4 * kb + 2 * jj + g;
      const int d = db * 32 + l32;
      vfr[slot] = *reinterpret_cast<const bf16x8*>(vl + d * KVT + 8 * (c ^ swz<VCPR>(d)));
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
  }
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

// Software-pipelined form: one wave per SIMD holding 96 query rows (three 32-row blocks) of one
// query head; the four waves of a workgroup (four query heads of one K/V head, or four row
// blocks of one head) share a 5-stage ring of 32-key K/V tiles. With no other wave on its SIMD,
// a wave hides its own softmax behind its MFMAs: each tile is six groups of 8 MFMAs (tile
// t + 1's S of block 0, tile t's P.V of block 0, the same for blocks 1 and 2), and every MFMA
// carries one score of a block's softmax, in the 16-key half that block's P.V needs next. The
// products, sums and max decisions are those of flash_attn_kernel, in the same order and with
// the same instructions, so the results are bitwise the same. Four S^T accumulators rotate over
// the blocks (tile t + 1 block x lands where tile t block x - 1's was), so the loop is unrolled
// by four tiles.
//
// The MFMAs and the softmax steps between them are inline assembly, one statement per MFMA, so
// that the compiler neither reorders them nor moves the P.V accumulators (held in AGPRs). The
// hazards the compiler no longer sees are covered by distance: a VALU instruction reads an S
// accumulator at least two groups after its last MFMA, a P word is read by an MFMA at least
// four instructions after its conversion, and the paths that touch accumulators sooner (the
// rare max raise, the tail mask, the epilogue) start with explicit wait states.
#define IRIS_EXP "v_exp_f32 %[x], %[f]\n\t"
#define IRIS_NEXT "v_fma_f32 %[fn], %[sn], %[k], -%[m]\n\t"
#define IRIS_PACK "v_cvt_pk_bf16_f32 %[w], %[x0], %[x]\n\t"
#define IRIS_ADD "v_add_f32 %[sum], %[sum], %[x]\n\t"

// One softmax step per MFMA. Step j of a 16-key half takes f = s_j * k - m (from the step
// before: no VALU instruction waits on the one just issued), issues x = exp2(f), the next
// step's fma (NEXT), the MFMA, then on odd steps the pair (x0, x) converted to a BF16 word w,
// and adds x to sum.
// S MFMA (VGPR accumulator c; ZERO: starting from zero, step 0)
template <bool ZERO, bool ODD, bool NEXT>
__device__ __forceinline__ void s_step(f32x16& c, const bf16x8& a, const bf16x8& b, float f, float sn, float k,
                                       float m, float& x, float& fn, float x0, unsigned& w, float& sum) {
  static_assert(!ZERO || (!ODD && NEXT), "the zero-start step is step 0");
  if constexpr (ZERO) {
    asm volatile(IRIS_EXP IRIS_NEXT "v_mfma_f32_32x32x16_bf16 %[c], %[a], %[b], 0\n\t" IRIS_ADD
                 : [c] "=&v"(c), [x] "=&v"(x), [fn] "=&v"(fn), [sum] "+v"(sum)
                 : [a] "v"(a), [b] "v"(b), [f] "v"(f), [sn] "v"(sn), [k] "s"(k), [m] "v"(m));
  } else if constexpr (!ODD) {
    asm volatile(IRIS_EXP IRIS_NEXT "v_mfma_f32_32x32x16_bf16 %[c], %[a], %[b], %[c]\n\t" IRIS_ADD
                 : [c] "+v"(c), [x] "=&v"(x), [fn] "=&v"(fn), [sum] "+v"(sum)
                 : [a] "v"(a), [b] "v"(b), [f] "v"(f), [sn] "v"(sn), [k] "s"(k), [m] "v"(m));
  } else if constexpr (NEXT) {
    asm volatile(IRIS_EXP IRIS_NEXT "v_mfma_f32_32x32x16_bf16 %[c], %[a], %[b], %[c]\n\t" IRIS_PACK IRIS_ADD
                 : [c] "+v"(c), [x] "=&v"(x), [fn] "=&v"(fn), [w] "=&v"(w), [sum] "+v"(sum)
                 : [a] "v"(a), [b] "v"(b), [f] "v"(f), [sn] "v"(sn), [k] "s"(k), [m] "v"(m), [x0] "v"(x0));
  } else {
    asm volatile(IRIS_EXP "v_mfma_f32_32x32x16_bf16 %[c], %[a], %[b], %[c]\n\t" IRIS_PACK IRIS_ADD
                 : [c] "+v"(c), [x] "=&v"(x), [w] "=&v"(w), [sum] "+v"(sum)
                 : [a] "v"(a), [b] "v"(b), [f] "v"(f), [x0] "v"(x0));
  }
}

// The P.V accumulators live in fixed AGPRs that only inline assembly touches: tile (db, qb)
// in a[16 k : 16 k + 15], k = 4 qb + db (the compiler allocates no AGPR of its own here).
#define IRIS_ACC_0 "a[0:15]"
#define IRIS_ACC_1 "a[16:31]"
#define IRIS_ACC_2 "a[32:47]"
#define IRIS_ACC_3 "a[48:63]"
#define IRIS_ACC_4 "a[64:79]"
#define IRIS_ACC_5 "a[80:95]"
#define IRIS_ACC_6 "a[96:111]"
#define IRIS_ACC_7 "a[112:127]"
#define IRIS_ACC_8 "a[128:143]"
#define IRIS_ACC_9 "a[144:159]"
#define IRIS_ACC_10 "a[160:175]"
#define IRIS_ACC_11 "a[176:191]"
#define IRIS_EL_0 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15
#define IRIS_EL_1 16, 17, 18, 19, 20, 21, 22, 23, 24, 25, 26, 27, 28, 29, 30, 31
#define IRIS_EL_2 32, 33, 34, 35, 36, 37, 38, 39, 40, 41, 42, 43, 44, 45, 46, 47
#define IRIS_EL_3 48, 49, 50, 51, 52, 53, 54, 55, 56, 57, 58, 59, 60, 61, 62, 63
#define IRIS_EL_4 64, 65, 66, 67, 68, 69, 70, 71, 72, 73, 74, 75, 76, 77, 78, 79
#define IRIS_EL_5 80, 81, 82, 83, 84, 85, 86, 87, 88, 89, 90, 91, 92, 93, 94, 95
#define IRIS_EL_6 96, 97, 98, 99, 100, 101, 102, 103, 104, 105, 106, 107, 108, 109, 110, 111
#define IRIS_EL_7 112, 113, 114, 115, 116, 117, 118, 119, 120, 121, 122, 123, 124, 125, 126, 127
#define IRIS_EL_8 128, 129, 130, 131, 132, 133, 134, 135, 136, 137, 138, 139, 140, 141, 142, 143
#define IRIS_EL_9 144, 145, 146, 147, 148, 149, 150, 151, 152, 153, 154, 155, 156, 157, 158, 159
#define IRIS_EL_10 160, 161, 162, 163, 164, 165, 166, 167, 168, 169, 170, 171, 172, 173, 174, 175
#define IRIS_EL_11 176, 177, 178, 179, 180, 181, 182, 183, 184, 185, 186, 187, 188, 189, 190, 191
#define IRIS_TILES(M) M(0) M(1) M(2) M(3) M(4) M(5) M(6) M(7) M(8) M(9) M(10) M(11)
#define IRIS_RD1(i, n) "v_accvgpr_read_b32 %" #i ", a" #n "\n\t"
#define IRIS_WR1(i, n) "v_accvgpr_write_b32 a" #n ", %" #i "\n\t"
#define IRIS_CL1(n) "a" #n
#define IRIS_RD16_(n0, n1, n2, n3, n4, n5, n6, n7, n8, n9, n10, n11, n12, n13, n14, n15) IRIS_RD1(0, n0) IRIS_RD1(1, n1) IRIS_RD1(2, n2) IRIS_RD1(3, n3) IRIS_RD1(4, n4) IRIS_RD1(5, n5) IRIS_RD1(6, n6) IRIS_RD1(7, n7) IRIS_RD1(8, n8) IRIS_RD1(9, n9) IRIS_RD1(10, n10) IRIS_RD1(11, n11) IRIS_RD1(12, n12) IRIS_RD1(13, n13) IRIS_RD1(14, n14) IRIS_RD1(15, n15)
#define IRIS_WR16_(n0, n1, n2, n3, n4, n5, n6, n7, n8, n9, n10, n11, n12, n13, n14, n15) IRIS_WR1(0, n0) IRIS_WR1(1, n1) IRIS_WR1(2, n2) IRIS_WR1(3, n3) IRIS_WR1(4, n4) IRIS_WR1(5, n5) IRIS_WR1(6, n6) IRIS_WR1(7, n7) IRIS_WR1(8, n8) IRIS_WR1(9, n9) IRIS_WR1(10, n10) IRIS_WR1(11, n11) IRIS_WR1(12, n12) IRIS_WR1(13, n13) IRIS_WR1(14, n14) IRIS_WR1(15, n15)
#define IRIS_CL16_(n0, n1, n2, n3, n4, n5, n6, n7, n8, n9, n10, n11, n12, n13, n14, n15) IRIS_CL1(n0), IRIS_CL1(n1), IRIS_CL1(n2), IRIS_CL1(n3), IRIS_CL1(n4), IRIS_CL1(n5), IRIS_CL1(n6), IRIS_CL1(n7), IRIS_CL1(n8), IRIS_CL1(n9), IRIS_CL1(n10), IRIS_CL1(n11), IRIS_CL1(n12), IRIS_CL1(n13), IRIS_CL1(n14), IRIS_CL1(n15)
#define IRIS_RD16(...) IRIS_RD16_(__VA_ARGS__)
#define IRIS_WR16(...) IRIS_WR16_(__VA_ARGS__)
#define IRIS_CL16(...) IRIS_CL16_(__VA_ARGS__)

// one P.V MFMA into accumulator tile K with one softmax step, as s_step
template <int K, bool ODD, bool NEXT>
__device__ __forceinline__ void o_step(const bf16x8& a, const bf16x8& b, float f, float sn, float k, float m, float& x,
                                       float& fn, float x0, unsigned& w, float& sum) {
#define IRIS_O_MFMA(kk) "v_mfma_f32_32x32x16_bf16 " IRIS_ACC_##kk ", %[a], %[b], " IRIS_ACC_##kk "\n\t"
#define IRIS_O_CASE(kk)                                                                                  \
  if constexpr (K == kk) {                                                                               \
    if constexpr (!ODD)                                                                                  \
      asm volatile(IRIS_EXP IRIS_NEXT IRIS_O_MFMA(kk) IRIS_ADD                                           \
                   : [x] "=&v"(x), [fn] "=&v"(fn), [sum] "+v"(sum)                                       \
                   : [a] "v"(a), [b] "v"(b), [f] "v"(f), [sn] "v"(sn), [k] "s"(k), [m] "v"(m)            \
                   : IRIS_CL16(IRIS_EL_##kk));                                                           \
    else if constexpr (NEXT)                                                                             \
      asm volatile(IRIS_EXP IRIS_NEXT IRIS_O_MFMA(kk) IRIS_PACK IRIS_ADD                                 \
                   : [x] "=&v"(x), [fn] "=&v"(fn), [w] "=&v"(w), [sum] "+v"(sum)                         \
                   : [a] "v"(a), [b] "v"(b), [f] "v"(f), [sn] "v"(sn), [k] "s"(k), [m] "v"(m), [x0] "v"(x0) \
                   : IRIS_CL16(IRIS_EL_##kk));                                                           \
    else                                                                                                 \
      asm volatile(IRIS_EXP IRIS_O_MFMA(kk) IRIS_PACK IRIS_ADD                                           \
                   : [x] "=&v"(x), [w] "=&v"(w), [sum] "+v"(sum)                                         \
                   : [a] "v"(a), [b] "v"(b), [f] "v"(f), [x0] "v"(x0)                                    \
                   : IRIS_CL16(IRIS_EL_##kk));                                                           \
  }
  IRIS_TILES(IRIS_O_CASE)
#undef IRIS_O_CASE
#undef IRIS_O_MFMA
}
// accumulator tile K <-> VGPRs
template <int K>
__device__ __forceinline__ f32x16 acc_read() {
  float e[16];
#define IRIS_RD_CASE(kk)                                                                                          \
  if constexpr (K == kk)                                                                                          \
    asm volatile(IRIS_RD16(IRIS_EL_##kk)                                                                          \
                 : "=v"(e[0]), "=v"(e[1]), "=v"(e[2]), "=v"(e[3]), "=v"(e[4]), "=v"(e[5]), "=v"(e[6]), "=v"(e[7]), \
                   "=v"(e[8]), "=v"(e[9]), "=v"(e[10]), "=v"(e[11]), "=v"(e[12]), "=v"(e[13]), "=v"(e[14]),       \
                   "=v"(e[15]));
  IRIS_TILES(IRIS_RD_CASE)
#undef IRIS_RD_CASE
  f32x16 v;
#pragma unroll
  for (int i = 0; i < 16; ++i) v[i] = e[i];
  return v;
}
template <int K>
__device__ __forceinline__ void acc_write(const f32x16& v) {
  float e[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) e[i] = v[i];
#define IRIS_WR_CASE(kk)                                                                                             \
  if constexpr (K == kk)                                                                                             \
    asm volatile(IRIS_WR16(IRIS_EL_##kk)                                                                             \
                 :                                                                                                   \
                 : "v"(e[0]), "v"(e[1]), "v"(e[2]), "v"(e[3]), "v"(e[4]), "v"(e[5]), "v"(e[6]), "v"(e[7]), "v"(e[8]), \
                   "v"(e[9]), "v"(e[10]), "v"(e[11]), "v"(e[12]), "v"(e[13]), "v"(e[14]), "v"(e[15])                 \
                 : IRIS_CL16(IRIS_EL_##kk));
  IRIS_TILES(IRIS_WR_CASE)
#undef IRIS_WR_CASE
}
// all twelve accumulator tiles to zero (0 x 0 + 0)
__device__ __forceinline__ void acc_zero_all() {
  const bf16x8 z = {};
#define IRIS_Z_CASE(kk) \
  asm volatile("v_mfma_f32_32x32x16_bf16 " IRIS_ACC_##kk ", %0, %0, 0" : : "v"(z) : IRIS_CL16(IRIS_EL_##kk));
  IRIS_TILES(IRIS_Z_CASE)
#undef IRIS_Z_CASE
}
#undef IRIS_EXP
#undef IRIS_NEXT
#undef IRIS_PACK
#undef IRIS_ADD

__device__ __forceinline__ void mfma_plain_zero(f32x16& c, const bf16x8& a, const bf16x8& b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(c) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma_plain(f32x16& c, const bf16x8& a, const bf16x8& b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b));
}
// wait states before VALU code touches the registers of MFMAs issued just before (the forms
// with operands also keep the compiler from moving the code that uses them above the wait)
#define IRIS_DRAIN "s_nop 15\n\ts_nop 15\n\ts_nop 15"
__device__ __forceinline__ void mfma_drain() { asm volatile(IRIS_DRAIN ::: "memory"); }
__device__ __forceinline__ void mfma_drain(f32x16& a, f32x16& b, f32x16& c) {
  asm volatile(IRIS_DRAIN : "+v"(a), "+v"(b), "+v"(c));
}
__device__ __forceinline__ void mfma_drain(unsigned (&w)[2][4]) {
  asm volatile(IRIS_DRAIN
               : "+v"(w[0][0]), "+v"(w[0][1]), "+v"(w[0][2]), "+v"(w[0][3]), "+v"(w[1][0]), "+v"(w[1][1]),
                 "+v"(w[1][2]), "+v"(w[1][3]));
}
#undef IRIS_DRAIN
template <int... I, typename F>
__device__ __forceinline__ void static_for_seq(std::integer_sequence<int, I...>, F&& f) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_seq(std::make_integer_sequence<int, N>{}, f);
}

template <int STAGES>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void flash_attn_pipe_kernel(AttnArgs p) {
  constexpr int QB = 3, KVT = 32;
  constexpr int TILE = KVT * kHd;
  constexpr int STAGE = 2 * TILE;
  constexpr int LOADS = KVT / 16;  // 1 KB loads per wave per operand per tile
  constexpr int LPW = 2 * LOADS;
  constexpr int VCPR = KVT / 8;
  constexpr int VRPL = 64 / VCPR;
  static_assert(STAGES >= 5 && (STAGES - 3) * LPW < 64, "ring depth");
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
  const int l32 = lane & 31;
  const int g = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int group = p.heads / p.kv_heads;
  const int h = kvh * group + hg * p.hpw + (w % p.hpw);
  const int q0 = qblk * p.rows_per_wg + (w / p.hpw) * 32 * QB;
  const long n_pad = p.n_pad;

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
  int k_off[LOADS], v_off[LOADS];
#pragma unroll
  for (int j = 0; j < LOADS; ++j) {
    const int kr = (w * LOADS + j) * 4 + (lane >> 4);
    k_off[j] = kr * kHd + 8 * ((lane & 15) ^ swz<16>(kr));
    const int vd = (w * LOADS + j) * VRPL + lane / VCPR;
    v_off[j] = vd * static_cast<int>(n_pad) + 8 * ((lane % VCPR) ^ swz<VCPR>(vd));
  }
  auto issue = [&](int t, int stage) {
    const __amdgpu_buffer_rsrc_t rk =
        __builtin_amdgcn_make_buffer_rsrc((void*)kh, (short)0, static_cast<int>(n_pad) * kHd * 2, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rv =
        __builtin_amdgcn_make_buffer_rsrc((void*)vh, (short)0, static_cast<int>(n_pad) * kHd * 2, kBufferFlags);
    bf16* kl = lds + stage * STAGE;
    bf16* vl = kl + TILE;
    // tile offsets as scalars (the compiler otherwise keeps them in VGPRs here and wraps each
    // load in a loop over lanes)
    const int so_k = __builtin_amdgcn_readfirstlane(t * KVT * kHd * 2);
    const int so_v = __builtin_amdgcn_readfirstlane(t * KVT * 2);
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      buffer_load_lds16(rk, kl + (w * LOADS + j) * 512, k_off[j] * 2, so_k);
      buffer_load_lds16(rv, vl + (w * LOADS + j) * 512, v_off[j] * 2, so_v);
    }
  };

  acc_zero_all();
  float m_run[QB], l_run[QB], sum[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) m_run[qb] = -INFINITY, l_run[qb] = 0.0f, sum[qb] = 0.0f;
  const float sl2 = p.scale_log2;
  const int n_tiles = (p.n + KVT - 1) / KVT;

  f32x16 sacc[QB];        // S^T of block x: tile t's until its max decision, then tile t + 1's
  unsigned pw[QB][2][4];  // P^T words of block x: [16-key half][word]
  constexpr int KD = 4;
  bf16x8 kf[KD];
  constexpr int VD = 6;
  bf16x8 vfr[VD];
  auto read_k = [&](const bf16* kl, int st, int slot) {
    kf[slot] = *reinterpret_cast<const bf16x8*>(kl + l32 * kHd + 8 * ((2 * st + g) ^ swz<16>(l32)));
  };
  auto read_v = [&](const bf16* vl, int i, int slot) {
    const int jj = i / 4, d = (i % 4) * 32 + l32;
    vfr[slot] = *reinterpret_cast<const bf16x8*>(vl + d * KVT + 8 * ((2 * jj + g) ^ swz<VCPR>(d)));
  };
  auto pword = [&](int x, int half) {
    return __builtin_bit_cast(bf16x8, (unsigned __attribute__((ext_vector_type(4)))){pw[x][half][0], pw[x][half][1],
                                                                                       pw[x][half][2], pw[x][half][3]});
  };

  // S group: tile t + 1's S^T of block y into sacc[y] (its K fragments 0 .. KD - 1 already
  // read), carrying half 1 of block x's probabilities (sacc[x] -> pw[x][1], added to sum[x]);
  // reads the next P.V group's first VD V^T fragments (vl) behind its last MFMAs.
  auto s_group = [&](auto yc, auto xc, const bf16* kl, const bf16* vl) {
    constexpr int y = decltype(yc)::value, x = decltype(xc)::value;
    static_assert(x != y, "the softmax reads another block's scores");
    float xv[8];
    float f = __builtin_fmaf(sacc[x][8], sl2, -m_run[x]);
    static_for<8>([&](auto stc) {
      constexpr int st = decltype(stc)::value;
      const float sn = sacc[x][8 + (st + 1) % 8];
      float fn;
      s_step<st == 0, st % 2 == 1, st < 7>(sacc[y], kf[st % KD], qf[y][st], f, sn, sl2, m_run[x], xv[st], fn,
                                           xv[(st + 7) % 8], pw[x][1][st / 2], sum[x]);
      f = fn;
      if constexpr (st + KD < 8) read_k(kl, st + KD, st % KD);
      if constexpr (st >= 8 - VD) read_v(vl, st - (8 - VD), st - (8 - VD));
    });
  };
  // P.V group: tile t's O^T += V^T P^T of block y (words pw[y]; V^T fragments 0 .. VD - 1
  // already read), carrying half 0 of block x's probabilities (sacc[x] -> pw[x][0], sum[x]
  // restarted); reads the next S group's first KD K fragments (kl) behind its last MFMAs.
  auto o_group = [&](auto yc, auto xc, const bf16* vl, const bf16* kl) {
    constexpr int y = decltype(yc)::value, x = decltype(xc)::value;
    static_assert(x != y, "the words read and the words written are another block's");
    const bf16x8 p0 = pword(y, 0), p1 = pword(y, 1);
    float xv[8];
    sum[x] = 0.0f;
    float f = __builtin_fmaf(sacc[x][0], sl2, -m_run[x]);
    static_for<8>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      const float sn = sacc[x][(i + 1) % 8];
      float fn;
      o_step<4 * y + i % 4, i % 2 == 1, i < 7>(vfr[i % VD], i < 4 ? p0 : p1, f, sn, sl2, m_run[x], xv[i], fn,
                                               xv[(i + 7) % 8], pw[x][0][i / 2], sum[x]);
      f = fn;
      if constexpr (i + VD < 8) read_v(vl, i + VD, i % VD);
      if constexpr (i >= 8 - KD) read_k(kl, i - (8 - KD), i - (8 - KD));
    });
  };
  // one half of block x's probabilities against m, written to its words and added to acc (the
  // prologue's and the max raise's path)
  auto probs_half = [&](int x, int half, float m, float& acc) {
    bf16x8 ph;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[x][8 * half + e], sl2, -m));
      ph[e] = from_f32<bf16>(v);
      acc += v;
    }
    const auto wv = __builtin_bit_cast(unsigned __attribute__((ext_vector_type(4))), ph);
#pragma unroll
    for (int e = 0; e < 4; ++e) pw[x][half][e] = wv[e];
  };
  // which lanes of block x need the max raise; the compare issues here, its result is read a
  // group later, so the wave never waits on it
  auto raise_mask = [&](int x) {
    const unsigned long long m = __ballot(!(sum[x] <= 256.0f));
    asm volatile("" ::"s"(m));
    return m;
  };
  // the lazy max raise of flash_attn_kernel for block x (m: raise_mask's lanes), then the sum
  // joins l
  auto settle = [&](auto xc, unsigned long long mask) {
    constexpr int x = decltype(xc)::value;
    if (__builtin_expect(mask != 0, 0)) {  // out of line: the common path takes no branch
      mfma_drain();
      const int need = !(sum[x] <= 256.0f);
      const int partner = __shfl_xor(need, 32);
      const bool up = need || partner;
      float mx = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[x][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = up ? fmaxf(m_run[x], mx * sl2) : m_run[x];
      const float alpha = __builtin_amdgcn_exp2f(m_run[x] - m_new);
      l_run[x] *= alpha;
      static_for<4>([&](auto dbc) {
        constexpr int k = 4 * x + decltype(dbc)::value;
        acc_write<k>(acc_read<k>() * alpha);
      });
      m_run[x] = m_new;
      float sm = 0.0f;
      probs_half(x, 0, m_new, sm);
      probs_half(x, 1, m_new, sm);
      sum[x] = sm;
      mfma_drain(pw[x]);  // the P.V MFMAs read these words next
    }
    l_run[x] += sum[x];
  };
  // keys >= n of tile t do not exist (its scores in sacc[x], just out of the MFMAs)
  auto mask_tail = [&](int x, int t) {
    mfma_drain(sacc[0], sacc[1], sacc[2]);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = t * KVT + 8 * (r >> 2) + 4 * g + (r & 3);
      if (key >= p.n) sacc[x][r] = -INFINITY;
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;

  // tile t: S(t+1)[0] | P.V(t)[0] | S(t+1)[1] | P.V(t)[1] | S(t+1)[2] | barrier | P.V(t)[2]; each
  // group carries one half of a block's softmax, and block x's max decision comes one group
  // after its sums are complete, before its P.V. TAIL: tile t + 1 is the last tile (masked when
  // partial); LAST: tile t is (the products of tile t + 1 are never used).
  auto tile = [&](int t, auto tailc, auto lastc) {
    constexpr bool TAIL = decltype(tailc)::value, LAST = decltype(lastc)::value;
    const bf16* kl = lds + ((t + 1) % STAGES) * STAGE;
    const bf16* vl = lds + (t % STAGES) * STAGE + TILE;
    const bf16* kl2 = lds + ((t + 2) % STAGES) * STAGE;
    const bool partial = TAIL && (t + 2) * KVT > p.n;

    s_group(I0{}, I1{}, kl, vl);
    const unsigned long long r1 = raise_mask(1);
    if (partial) mask_tail(0, t + 1);
    o_group(I0{}, I2{}, vl, kl);
    settle(I1{}, r1);
    s_group(I1{}, I2{}, kl, vl);
    const unsigned long long r2 = raise_mask(2);
    if (partial) mask_tail(1, t + 1);
    o_group(I1{}, I0{}, vl, kl);
    settle(I2{}, r2);
    s_group(I2{}, I0{}, kl, vl);
    const unsigned long long r0 = raise_mask(0);
    if (partial) mask_tail(2, t + 1);
    // tile t + 2 visible for the next tile's first group (tiles up to t + STAGES - 2 were
    // issued); stage (t - 1) % STAGES no longer read: refilled with tile t + STAGES - 1 (past the
    // end the last tile again, into a stage nothing reads, so every tile waits and loads alike)
    wait_vmcnt<(STAGES - 4) * LPW>();
    __builtin_amdgcn_s_barrier();
    issue(min(t + STAGES - 1, n_tiles - 1), (t + STAGES - 1) % STAGES);
    o_group(I2{}, I1{}, vl, kl2);
    if constexpr (!LAST) settle(I0{}, r0);
  };

#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s) issue(min(s, n_tiles - 1), s);
  wait_vmcnt<(STAGES - 3) * LPW>();  // tiles 0 and 1 landed
  __builtin_amdgcn_s_barrier();
  // tile 0's S^T; block 0's probabilities and max decision, block 1's first half; the first K
  // fragments of the first group
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      const bf16x8 kfr = *reinterpret_cast<const bf16x8*>(lds + l32 * kHd + 8 * ((2 * st + g) ^ swz<16>(l32)));
      if (st == 0)
        mfma_plain_zero(sacc[qb], kfr, qf[qb][0]);
      else
        mfma_plain(sacc[qb], kfr, qf[qb][st]);
    }
  }
  mfma_drain(sacc[0], sacc[1], sacc[2]);
  if (KVT > p.n) {
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) mask_tail(qb, 0);
  }
  probs_half(0, 0, m_run[0], sum[0]);
  probs_half(0, 1, m_run[0], sum[0]);
  settle(I0{}, raise_mask(0));
  probs_half(1, 0, m_run[1], sum[1]);
#pragma unroll
  for (int st = 0; st < KD; ++st) read_k(lds + STAGE, st, st);
  using F = std::false_type;
  using T = std::true_type;
  int t = 0;
  for (; t + 2 < n_tiles; ++t) tile(t, F{}, F{});
  if (t + 1 < n_tiles) tile(t++, T{}, F{});
  tile(t, F{}, T{});
  wait_vmcnt<0>();  // the repeated loads past the last tile land before the workgroup ends
  mfma_drain();

  static_for<QB>([&](auto qbc) {
    constexpr int qb = decltype(qbc)::value;
    f32x16 oq[4];
    static_for<4>([&](auto dbc) { oq[decltype(dbc)::value] = acc_read<4 * qb + decltype(dbc)::value>(); });
    store_row(p, oq, l_run[qb], b, h, q0 + qb * 32 + l32, g);
  });
}

struct Variant {
  int qb, stages, kvt;
  bool staged;
  int nw = 4;
  bool pipe = false;
};
// 0: 32 query rows per wave, 64-key tiles staged through registers; 1: the same with 32-key
// tiles; 2: 64-key tiles, 2-stage ring; 3: 32-key tiles, 3-stage ring; 4: 32-key
// tiles in a 3-stage ring shared by twelve waves (four query heads x three row blocks).
// (Measured and dropped: twelve-wave rings of 4 and 6 stages (1-2% slower than 3), eight of the
// twelve waves fetching instead of four (2% slower), 64-key tiles at twelve waves (spills); an eight-wave ping-pong of MFMA and softmax phases, 1.8x slower at the
// trunk shape; a software-pipelined wave issuing tile t - 1's P.V MFMAs around tile t's softmax,
// no faster than variant 1; a twelve-wave form issuing tile t + 1's S MFMAs between tile t's
// softmax instructions (4-stage ring), 1% faster than variant 4; 64- and 96-row waves at one
// wave per SIMD, 1.5-1.9x slower.)
constexpr Variant kVariants[] = {{1, 2, 64, true},  {1, 2, 32, true},      {1, 2, 64, false},
                                 {1, 3, 32, false}, {1, 3, 32, false, 12}, {3, 8, 32, false, 4, true}};
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
  // ring (one per CU; 230 of them cover a 4352-token sequence) when their rounds over the CUs
  // are at least 80% full, 9-11% faster than variant 1 there; else 32-key tiles staged through
  // registers in three 4-wave workgroups per CU (variant 1: 168 VGPRs; small grids spread
  // over more CUs). One query head per K/V head (the pixel stage): 64-key tiles in a
  // 2-stage ring. Each measured fastest at its shapes.
  int variant = g_attn_variant;
  if (variant < 0) {
    variant = group >= 4 ? 1 : 2;
    if (group >= 4) {
      const int cus = device_cus();
      const long wide = static_cast<long>(batch) * kv_heads * (group / 4) * ((n + 95) / 96);
      const long rounds = (wide + cus - 1) / cus;
      if (wide >= 0.8 * rounds * cus) variant = 4;
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
    default:
      flash_attn_pipe_kernel<8><<<grid, 256, 0, stream>>>(args);
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
