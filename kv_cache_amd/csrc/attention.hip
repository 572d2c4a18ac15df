// GQA-native sparse gather attention over selected KV blocks (bf16 or fp16
// q/K/V/output, fp32 softmax and accumulation), one launch per call.
//
// The reference expands K/V to every query head (evaluate_qwen3_top2_head_
// limit3_ppl.py:6248-6251) and then gathers per head (EV:4490-4502, kernel
// qabs_cuda_kernels.py:335-419).  Here the G query heads of a KV head share
// one pass over the selected rows, so every selected K/V row is read from HBM
// once (512 bytes per token at D = 128).
//
// Work split: slot s of a row is token (block_ids[s / block] * block +
// s % block).  A workgroup (4 waves) owns a contiguous range of slots of one
// (sequence, KV head) row; its waves take chunks of slots in turn (chunk c of
// wave w is the workgroup's chunk 4c + w).  While a wave computes chunk c,
// the K/V loads of chunk c+1 and the block ids of chunk c+2 are in flight;
// the chunk loop is unrolled at compile time and every load is issued
// without a branch, so each wait covers exactly the loads it needs.
//
// Two chunk kernels share that frame.  sparse_attn_mfma_kernel (G >= 2) runs
// QK and P.V on the matrix cores over 16-slot chunks (its comment has the
// operand layouts).  sparse_attn_kernel (G = 1) runs them on the VALU: 16
// lanes share a token (lane 16g + c holds channels 8c..8c+7 of the token of
// slot 4i + g in step i, so each load instruction reads four whole 256-byte
// rows), QK is v_dot2_f32_bf16 (v_dot2_f32_f16 for fp16) on the packed
// channel pairs and a 16-lane DPP sum, softmax runs in the log2 domain with a
// running maximum per 16-lane token group, P.V accumulates in fp32, and a wave combines its four token
// groups with the gfx950 lane swaps (v_permlane16_swap / v_permlane32_swap).
//
// A workgroup combines its waves through LDS into (max, sum, weighted V) per
// head.  A row that fits one workgroup writes its output directly.
// Otherwise every workgroup publishes its partial with device-coherent
// stores (relaxed agent-scope atomic stores: global_store sc1, written
// through the XCD's L2), waits for them to complete, and takes a ticket; the
// row's last workgroup reads all partials back with device-coherent loads
// (sc1), every load of a batch in flight at once, and writes the output.
// No release / acquire fence is used: on gfx950 those write back and
// invalidate the whole L2 of the XCD (buffer_wbl2 / buffer_inv).
#include <mutex>

#include "common.h"
#include "attend.h"

namespace qkv {
namespace {

// SELV > 0: the row's block ids are not given; every workgroup of the row
// selects the n_sel largest of its block maxima (bmax row r at bmax +
// r*bmax_ld, lowest index wins ties, ascending) into LDS first -- the
// selection of qkv_topk, repeated per split instead of launched separately,
// with SELV keys per thread (rows of at most 64*NW*SELV blocks; the selection's
// latency grows with SELV).  The row's first workgroup also writes it to
// sel_out (when given).
template <int G, int NI, int ITERS, int SELV, int NW, bool F16>
__global__ __launch_bounds__(64 * NW, QKV_ATTN_WG_PER_CU * 4 / NW) void sparse_attn_kernel(
    const uint16_t* __restrict__ query, const uint16_t* __restrict__ key,
    const uint16_t* __restrict__ value, int64_t sb, int64_t sh, int64_t st, int q_heads,
    int kv_heads, int tokens, const int32_t* __restrict__ block_ids, int n_sel, int block,
    int nb, float scale_log2, int nsplit, float* __restrict__ ws_acc, float* __restrict__ ws_ml,
    uint32_t* __restrict__ tickets, uint16_t* __restrict__ out, const float* __restrict__ bmax,
    int64_t bmax_ld, int32_t* __restrict__ sel_out, int kv_div, int n_prot, int sink_end, int recent_start,
    int rec_begin, int n_rec, int self_tok) {
  constexpr int CH = 4 * NI;               // token slots per wave chunk
  constexpr int NT = 64 * NW;              // threads per workgroup
  static_assert(CH <= 64, "one slot per lane when resolving token ids");

  __shared__ float red_acc[NW][G][kD];   // per wave weighted V
  __shared__ float red_m[NW][G], red_l[NW][G];
  __shared__ int last_flag;
  constexpr bool SEL = SELV > 0;
  __shared__ int32_t sel_lds[SEL ? NT * SELV : 1];

  const int r = blockIdx.y, split = blockIdx.x;
  const int b = r / kv_heads, j = r - b * kv_heads;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int grp = lane >> 4, cc = lane & 15;
  const float ninf = -__builtin_huge_valf();
  if constexpr (SEL) {
    select_row<SEL ? SELV : 1, false, NW>(bmax + static_cast<int64_t>(r) * bmax_ld, nb, n_sel, sel_lds);
    if (sel_out && split == 0)
      for (int i = tid; i < n_sel; i += NT) sel_out[static_cast<int64_t>(r) * n_sel + i] = sel_lds[i];
  }
  const int n_blk_slots = n_sel * block;
  const RowSlots rs{SEL ? sel_lds : block_ids + static_cast<int64_t>(r) * n_sel, n_blk_slots, n_blk_slots + n_prot,
                    block, nb, tokens, sink_end, recent_start, rec_begin, n_rec, self_tok};

  // Slot of this lane in chunk c (meaningful for lane < CH).
  const int wg_base = split * (NW * CH * ITERS);
  auto slot_of = [&](int c) -> int { return wg_base + (NW * c + wave) * CH + lane; };
  auto load_id = [&](int c) -> int { return rs.id_of(slot_of(c), lane < CH); };
  auto token_of = [&](int c, int id) -> int { return rs.token_of(slot_of(c), id); };
  // Token of slot 4i + grp (the lane's token in step i), from lane 4i + grp.
  auto spread = [&](int my_tok, int (&tk)[NI]) {
#pragma unroll
    for (int i = 0; i < NI; ++i) tk[i] = __builtin_amdgcn_ds_bpermute((4 * i + grp) << 2, my_tok);
  };

  const int jk = j / kv_div;   // the K/V head this row reads
  const uint16_t* kb = key + b * sb + jk * sh + cc * 8;
  const uint16_t* vb = value + b * sb + jk * sh + cc * 8;
  // Invalid slots load token 0 of the row (in bounds) and are masked later.
  auto load_kv = [&](const int (&tk)[NI], uint4 (&kx)[NI], uint4 (&vx)[NI]) {
#pragma unroll
    for (int i = 0; i < NI; ++i) kx[i] = ld_nt(kb + static_cast<int64_t>(max(tk[i], 0)) * st);
#pragma unroll
    for (int i = 0; i < NI; ++i) vx[i] = ld_nt(vb + static_cast<int64_t>(max(tk[i], 0)) * st);
  };

  uint4 qx[G];
  const uint16_t* qrow = query + (static_cast<int64_t>(b) * q_heads + j * G) * kD + cc * 8;
#pragma unroll
  for (int h = 0; h < G; ++h) qx[h] = *reinterpret_cast<const uint4*>(qrow + h * kD);
  // G = 2, 4: each lane of a 16-lane token group ends up with the full QK sum
  // of one head, own = 2*b0 + b1 (G = 4) or b0 (G = 2) from the lane's low
  // bits.  Register k holds head own ^ k, so the pairwise reduce-scatter over
  // lanes l^1 and l^2 needs no per-lane select: the partner's register k + G/2
  // (step 1) and register 1 (step 2, G = 4) hold this lane's head.
  constexpr bool kScatter = G == 2 || G == 4;
  const int own = G == 4 ? 2 * (lane & 1) + ((lane >> 1) & 1) : (lane & 1);
  if constexpr (kScatter) {
    uint4 qp[G];
#pragma unroll
    for (int k = 0; k < G; ++k) {
      qp[k] = qx[0];
#pragma unroll
      for (int h = 1; h < G; ++h)
        if ((own ^ k) == h) qp[k] = qx[h];
    }
#pragma unroll
    for (int k = 0; k < G; ++k) qx[k] = qp[k];
  }

  // Running state of this lane's token group: max (log2 domain), sum, P.V.
  float m[G], l[G], acc[G][8];
  float m_own = ninf, l_own = 0.0f;   // scattered path: running max / sum of head `own`
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = ninf;
    l[h] = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[h][c] = 0.0f;
  }

  // Head value of the scattered path from the quad lane that owns head h.
  auto from_head = [](float v, int h) -> float {
    const int o = G == 4 ? (h >> 1) | ((h & 1) << 1) : h;   // quad lane of head h
    return o == 0 ? dpp_f<0x00>(v) : o == 1 ? dpp_f<0x55>(v) : o == 2 ? dpp_f<0xAA>(v) : dpp_f<0xFF>(v);
  };
  auto compute_scatter = [&](const int (&tk)[NI], const uint4 (&kx)[NI], const uint4 (&vx)[NI]) {
    float s[NI];
    float cm = ninf;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      float r[G];
#pragma unroll
      for (int k = 0; k < G; ++k) {
        float a = dot2_half<F16>(qx[k].x, kx[i].x, 0.0f);
        a = dot2_half<F16>(qx[k].y, kx[i].y, a);
        a = dot2_half<F16>(qx[k].z, kx[i].z, a);
        r[k] = dot2_half<F16>(qx[k].w, kx[i].w, a);
      }
      float y;
      if constexpr (G == 4) {
        const float x0 = r[0] + dpp_f<0xB1>(r[2]);   // lanes l, l^1
        const float x1 = r[1] + dpp_f<0xB1>(r[3]);
        y = x0 + dpp_f<0x4E>(x1);                    // lanes l, l^2
      } else {
        y = r[0] + dpp_f<0xB1>(r[1]);
        y = y + dpp_f<0x4E>(y);
      }
      // Rotations by 8 then 4 give the 4 lanes of a head the same sum, bit for bit.
      y = y + dpp_f<0x128>(y);
      y = y + dpp_f<0x124>(y);
      s[i] = tk[i] >= 0 ? y * scale_log2 : ninf;
      cm = fmaxf(cm, s[i]);
    }
    const float mn = fmaxf(m_own, cm);
    const float ms = (mn == ninf) ? 0.0f : mn;
    const float al = exp2f(m_own - ms);   // 0 while m_own = -inf
    l_own *= al;
    m_own = mn;
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float ah = from_head(al, h);
#pragma unroll
      for (int c = 0; c < 8; ++c) acc[h][c] *= ah;
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      float v[8];
      v[0] = half_lo<F16>(vx[i].x); v[1] = half_hi<F16>(vx[i].x);
      v[2] = half_lo<F16>(vx[i].y); v[3] = half_hi<F16>(vx[i].y);
      v[4] = half_lo<F16>(vx[i].z); v[5] = half_hi<F16>(vx[i].z);
      v[6] = half_lo<F16>(vx[i].w); v[7] = half_hi<F16>(vx[i].w);
      const float p = exp2f(s[i] - ms);   // 0 for masked slots
      l_own += p;
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float ph = from_head(p, h);
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[h][c] = __builtin_fmaf(ph, v[c], acc[h][c]);
      }
    }
    pin(l_own);
#pragma unroll
    for (int h = 0; h < G; ++h) {
#pragma unroll
      for (int c = 0; c < 8; ++c) pin(acc[h][c]);
    }
  };
  auto compute = [&](const int (&tk)[NI], const uint4 (&kx)[NI], const uint4 (&vx)[NI]) {
    if constexpr (kScatter) {
      compute_scatter(tk, kx, vx);
      return;
    }
    float s[G][NI], cm[G];
#pragma unroll
    for (int h = 0; h < G; ++h) cm[h] = ninf;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float a = dot2_half<F16>(qx[h].x, kx[i].x, 0.0f);
        a = dot2_half<F16>(qx[h].y, kx[i].y, a);
        a = dot2_half<F16>(qx[h].z, kx[i].z, a);
        a = dot2_half<F16>(qx[h].w, kx[i].w, a);
        a = row16_sum(a) * scale_log2;
        s[h][i] = tk[i] >= 0 ? a : ninf;
        cm[h] = fmaxf(cm[h], s[h][i]);
      }
    }
    // Rescale the group's state to the new maximum.  A group that has seen no
    // valid token keeps m = -inf; its exponent base is 0 so every p is 0.
    float ms[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float mn = fmaxf(m[h], cm[h]);
      ms[h] = (mn == ninf) ? 0.0f : mn;
      const float al = exp2f(m[h] - ms[h]);   // 0 while m = -inf
      l[h] *= al;
#pragma unroll
      for (int c = 0; c < 8; ++c) acc[h][c] *= al;
      m[h] = mn;
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      float v[8];
      v[0] = half_lo<F16>(vx[i].x); v[1] = half_hi<F16>(vx[i].x);
      v[2] = half_lo<F16>(vx[i].y); v[3] = half_hi<F16>(vx[i].y);
      v[4] = half_lo<F16>(vx[i].z); v[5] = half_hi<F16>(vx[i].z);
      v[6] = half_lo<F16>(vx[i].w); v[7] = half_hi<F16>(vx[i].w);
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float p = exp2f(s[h][i] - ms[h]);   // 0 for masked slots
        l[h] += p;
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[h][c] = __builtin_fmaf(p, v[c], acc[h][c]);
      }
    }
    // The chunk is done here: its K/V registers are free for the next one.
#pragma unroll
    for (int h = 0; h < G; ++h) {
      pin(l[h]);
#pragma unroll
      for (int c = 0; c < 8; ++c) pin(acc[h][c]);
    }
  };

  // Chunk pipeline: K/V of chunks c+1 .. c+P and the ids of chunk c+P+1 in
  // flight while chunk c computes (P = kDepth - 1).
  constexpr int P = kDepth - 1;
  uint4 kx[kDepth][NI], vx[kDepth][NI];
  int tk[kDepth][NI];
  int id_next = -1;
  {
    int id = load_id(0);
#pragma unroll
    for (int c = 0; c < P && c < ITERS; ++c) {
      const int idn = c + 1 < ITERS ? load_id(c + 1) : -1;
      spread(token_of(c, id), tk[c]);
      load_kv(tk[c], kx[c], vx[c]);
      id = idn;
    }
    id_next = id;
  }
  // Chunk c+P's loads go out only after chunk c-1 is computed (zero_after on
  // its state), so at most kDepth chunks of K/V occupy registers; the
  // scheduling barriers keep them ahead of chunk c's arithmetic.
  // (Register buffer u holds chunks u, u + kDepth, ...: the inner loop keeps
  // every buffer index a constant even where the outer one stays a loop.)
#pragma unroll
  for (int c0 = 0; c0 < ITERS; c0 += kDepth) {
#pragma unroll
    for (int u = 0; u < kDepth; ++u) {
      const int c = c0 + u;
      if (c >= ITERS) break;
      const int nxt = (u + P) % kDepth;
      __builtin_amdgcn_sched_barrier(0);
      if (c + P < ITERS) {
        const int dz = c > 0 ? zero_after(kScatter ? l_own : l[0]) : 0;
        const int tn = token_of(c + P, id_next + dz);
        if (c + P + 1 < ITERS) id_next = load_id(c + P + 1 + dz);
        spread(tn, tk[nxt]);
        load_kv(tk[nxt], kx[nxt], vx[nxt]);
      }
      __builtin_amdgcn_sched_barrier(0);
      compute(tk[u], kx[u], vx[u]);
    }
  }

  if constexpr (kScatter) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      m[h] = from_head(m_own, h);
      l[h] = from_head(l_own, h);
    }
  }
  // Combine the wave's four token groups: common max, rescale, sum.
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const float mw = max_x32(max_x16(m[h]));
    const float f = (m[h] == ninf) ? 0.0f : exp2f(m[h] - mw);
    l[h] = sum_x32(sum_x16(l[h] * f));
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[h][c] = sum_x32(sum_x16(acc[h][c] * f));
    m[h] = mw;
  }
  if (grp == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
#pragma unroll
      for (int c = 0; c < 8; ++c) red_acc[wave][h][cc * 8 + c] = acc[h][c];
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      red_m[wave][h] = m[h];
      red_l[wave][h] = l[h];
    }
  }
  __syncthreads();

  finish_workgroup<G, NW, F16>(red_acc, red_m, red_l, last_flag, r, split, nsplit,
                          out + (static_cast<int64_t>(b) * q_heads + j * G) * kD, ws_acc, ws_ml, tickets);
}

template <int G, int ITERS, int SELV, bool F16>
__global__ __launch_bounds__(256, QKV_ATTN_WG_PER_CU) void sparse_attn_mfma_kernel(const AttnArgs a) {
  attend_mfma<G, ITERS, SELV, (SELV > 0 ? kIdsSelect : kIdsGiven), F16>(a, blockIdx.y, blockIdx.x);
}

// 4-token steps per wave chunk: 8 while the G heads' state leaves room for
// two chunks of K/V in registers, 4 above that.
constexpr int ni_for(int64_t g) { return g <= 2 ? 8 : 4; }

// Group sizes from QKV_ATTN_MFMA_MIN_G up run sparse_attn_mfma_kernel.
// Measured with 256 selected blocks of 16 on 256 rows (cfg3's bytes), random
// block ids: VALU kernel G = 1 / 2 / 4 / 8: 91.2 / 95.8 / 101.0 / 199.3 us;
// MFMA kernel 94.8 / 95.4 / 97.0 / 100.0 us.  G = 1 keeps the VALU kernel,
// whose QK and P.V are a few instructions per token there.
#ifndef QKV_ATTN_MFMA_MIN_G
#define QKV_ATTN_MFMA_MIN_G 2
#endif
constexpr bool mfma_for(int64_t g) { return g >= QKV_ATTN_MFMA_MIN_G; }

// Slots a workgroup covers per chunk round.
constexpr int64_t per_iter_for(int64_t g) { return mfma_for(g) ? 4 * 16 : kWaves * 4 * ni_for(g); }

// Chunks per wave: doubled (up to max_iters_for) while the grid keeps
// QKV_ATTN_TARGET_WGS workgroups, so long selections take few splits per
// row.  Measured at cfg2 (64 rows x 2048 slots): 256 workgroups of 4 chunks
// per wave 18.0 us, 1024 workgroups of 1 chunk 20.4 us, 128 of 8 22.2 us.
// VALU kernel: G = 8 stops at 8 chunks (its 16-chunk variant does not fit
// the registers); G = 4 goes on to 32: at cfg3 (256 rows x 4096 slots) 512
// workgroups of 32 chunks, all resident at two per CU, take 101.4 us against
// 106.0 us for 1024 workgroups of 16 chunks in two rounds.  The MFMA kernel's
// 16-slot chunks go to 32 for every G.
constexpr int max_iters_for(int64_t g) { return mfma_for(g) ? 32 : g >= 8 ? 8 : g == 4 ? 32 : 16; }

// Doubling stops once one workgroup covers the whole row: further chunks
// would only walk empty slots.
int iters_for(int64_t rows, int64_t n_slots, int64_t g) {
  return chunk_rounds(rows, n_slots, per_iter_for(g), max_iters_for(g));
}

int64_t splits_for(int64_t rows, int64_t n_slots, int64_t g) {
  return cdiv(n_slots, per_iter_for(g) * iters_for(rows, n_slots, g));
}


template <int GG, int IT, int SS, bool FF>
void launch_attn(dim3 grid, hipStream_t st, const AttnArgs& a) {
#define QKV_ATTN_ARGS                                                                                          \
  a.q, a.k, a.v, a.sb, a.sh, a.st, a.q_heads, a.kv_heads, a.tokens, a.block_ids, a.n_sel, a.block, a.nb,    \
      a.scale_log2, a.nsplit, a.ws_acc, a.ws_ml, a.tickets, a.out, a.bmax, a.bmax_ld, a.sel_out, a.kv_div,   \
      a.n_prot, a.sink_end, a.recent_start, a.rec_begin, a.n_rec, a.self_tok
  if constexpr (mfma_for(GG))
    sparse_attn_mfma_kernel<GG, IT, SS, FF><<<grid, 256, 0, st>>>(a);
  else
    sparse_attn_kernel<GG, ni_for(GG), IT, SS, kWaves, FF><<<grid, 64 * kWaves, 0, st>>>(QKV_ATTN_ARGS);
#undef QKV_ATTN_ARGS
}

// The selection's keys per thread: 8 (at 4 waves) for rows of <= 2048
// blocks, 16 above.
template <int GG, int IT, bool FF>
void launch_attn_sel(dim3 grid, hipStream_t st, const AttnArgs& a, bool sel) {
  constexpr int W = mfma_for(GG) ? 4 : kWaves;
  if (!sel) launch_attn<GG, IT, 0, FF>(grid, st, a);
  else if (a.nb <= 2048) launch_attn<GG, IT, 32 / W, FF>(grid, st, a);
  else launch_attn<GG, IT, 64 / W, FF>(grid, st, a);
}

template <int GG, bool FF>
void launch_attn_g(int iters, dim3 grid, hipStream_t st, const AttnArgs& a, bool sel) {
  constexpr int MAXI = max_iters_for(GG);
  switch (iters) {
    case 1: launch_attn_sel<GG, 1, FF>(grid, st, a, sel); break;
    case 2: launch_attn_sel<GG, 2, FF>(grid, st, a, sel); break;
    case 4: launch_attn_sel<GG, 4, FF>(grid, st, a, sel); break;
    case 8: launch_attn_sel<GG, 8, FF>(grid, st, a, sel); break;
    case 16: if constexpr (MAXI >= 16) launch_attn_sel<GG, 16, FF>(grid, st, a, sel); break;
    default: if constexpr (MAXI >= 32) launch_attn_sel<GG, 32, FF>(grid, st, a, sel); break;
  }
}

template <bool FF>
void launch_attn_dt(int64_t g, int iters, dim3 grid, hipStream_t st, const AttnArgs& a, bool sel) {
  switch (g) {
    case 1: launch_attn_g<1, FF>(iters, grid, st, a, sel); break;
    case 2: launch_attn_g<2, FF>(iters, grid, st, a, sel); break;
    case 4: launch_attn_g<4, FF>(iters, grid, st, a, sel); break;
    default: launch_attn_g<8, FF>(iters, grid, st, a, sel); break;
  }
}

}  // namespace
}  // namespace qkv

using namespace qkv;

QKV_EXPORT int64_t qkv_sparse_attention_workspace_bytes(int64_t batch, int64_t q_heads,
                                                        int64_t kv_heads, int64_t head_dim,
                                                        int64_t n_sel, int64_t block) {
  if (batch <= 0 || kv_heads <= 0 || q_heads % kv_heads || head_dim != kD || n_sel <= 0 ||
      block <= 0 || n_sel * block >= (int64_t(1) << 30))
    return -1;
  const int64_t g = q_heads / kv_heads;
  return 4 * (kTicketWords + attention_partial_words(batch * kv_heads, n_sel * block, g, per_iter_for(g),
                                                     max_iters_for(g)));
}

namespace {

// Shared argument checks and launch of both entry points; sel selects the
// in-kernel selection from bmax (block_ids unused), else block_ids is read.
int launch_attention(const char* what, const void* query, const void* key, const void* value,
                     const int64_t* kv_strides, int64_t batch, int64_t q_heads, int64_t kv_heads,
                     int64_t tokens, int64_t head_dim, const int32_t* block_ids, const float* bmax,
                     int64_t bmax_ld, int32_t* sel_out, int64_t n_sel, int64_t block, float scaling,
                     float* workspace, int64_t workspace_bytes, void* out, int dtype, void* stream,
                     int kv_div = 1, int64_t protect_sink = 0, int64_t protect_recent = 0, bool keep_self = false) {
  const bool sel = bmax != nullptr;
  if (!query || !key || !value || !kv_strides || !(sel || block_ids) || !workspace || !out)
    return fail(QKV_ERR_INVALID, "%s: null pointer", what);
  bool f16;
  if (int rc = half_dtype(dtype, what, &f16)) return rc;
  if (head_dim != kD) return fail(QKV_ERR_UNSUPPORTED, "%s: head_dim must be 128", what);
  if (batch <= 0 || kv_heads <= 0 || q_heads % kv_heads)
    return fail(QKV_ERR_INVALID, "%s: q_heads must be a multiple of kv_heads", what);
  const int64_t g = q_heads / kv_heads;
  if (g != 1 && g != 2 && g != 4 && g != 8)
    return fail(QKV_ERR_UNSUPPORTED, "%s: group size %lld not built", what, (long long)g);
  if (batch * kv_heads > 65535) return fail(QKV_ERR_INVALID, "%s: too many rows", what);
  if (tokens <= 0 || tokens >= (int64_t(1) << 31) || n_sel <= 0 || block <= 0 ||
      n_sel * block >= (int64_t(1) << 30))
    return fail(QKV_ERR_INVALID, "%s: need tokens > 0, n_sel > 0, block > 0, n_sel * block < 2^30", what);
  if (!aligned(query, 16) || !aligned(key, 16) || !aligned(value, 16) ||
      (kv_strides[0] | kv_strides[1] | kv_strides[2]) % 8)
    return fail(QKV_ERR_INVALID, "%s: q/K/V rows must be 16-byte aligned", what);
  const int nb = static_cast<int>(cdiv(tokens, block));
  if (sel) {
    if (nb > kSelMaxBlocks)
      return fail(QKV_ERR_UNSUPPORTED, "%s: at most %d blocks (got %d); select with qkv_topk_ws first", what,
                  kSelMaxBlocks, nb);
    if (n_sel > nb || bmax_ld < nb) return fail(QKV_ERR_INVALID, "%s: need n_sel <= blocks <= bmax_ld", what);
  }
  // Protected tokens (EV:2938-2982): the sink range [0, sink_end), the
  // recent range [rec_begin, tokens) and the current token `tokens` (the
  // selection covers the history [0, tokens); K/V then hold tokens + 1 rows).
  const int64_t sink_end = protect_sink > 0 ? std::min(protect_sink, tokens) : 0;
  const int64_t recent_start = protect_recent > 0 ? std::max<int64_t>(0, tokens - protect_recent) : tokens;
  const int64_t rec_begin = std::max(recent_start, sink_end);
  const int64_t n_rec = protect_recent > 0 && rec_begin < tokens ? tokens - rec_begin : 0;
  const int64_t n_prot = sink_end + n_rec + (keep_self ? 1 : 0);
  if (n_sel * block + n_prot >= (int64_t(1) << 30)) return fail(QKV_ERR_INVALID, "%s: too many slots", what);
  // the workspace of a selection of n_sel + ceil(n_prot / block) blocks covers the protected slots
  const int64_t need = qkv_sparse_attention_workspace_bytes(batch, q_heads, kv_heads, head_dim,
                                                            n_sel + cdiv(n_prot, block), block);
  if (workspace_bytes < need)
    return fail(QKV_ERR_INVALID, "%s: workspace needs %lld bytes, got %lld", what, (long long)need,
                (long long)workspace_bytes);
  const int64_t rows = batch * kv_heads;
  const int64_t n_slots = n_sel * block + n_prot;
  const int iters = iters_for(rows, n_slots, g);
  const int64_t nsplit = splits_for(rows, n_slots, g);
  if (nsplit > 65535) return fail(QKV_ERR_INVALID, "%s: too many selected blocks", what);
  uint32_t* tickets = reinterpret_cast<uint32_t*>(workspace);
  float* ws_acc = workspace + kTicketWords;
  float* ws_ml = ws_acc + rows * nsplit * g * kD;
  const float scale_log2 = scaling * 1.4426950408889634f;
  hipStream_t st = static_cast<hipStream_t>(stream);
  dim3 grid(static_cast<unsigned>(nsplit), static_cast<unsigned>(rows));
  const uint16_t* q = static_cast<const uint16_t*>(query);
  const uint16_t* k = static_cast<const uint16_t*>(key);
  const uint16_t* v = static_cast<const uint16_t*>(value);
  uint16_t* o = static_cast<uint16_t*>(out);
  const AttnArgs a{q, k, v, kv_strides[0], kv_strides[1], kv_strides[2], static_cast<int>(q_heads),
                   static_cast<int>(kv_heads), static_cast<int>(tokens), block_ids, static_cast<int>(n_sel),
                   static_cast<int>(block), nb, scale_log2, static_cast<int>(nsplit), ws_acc, ws_ml, tickets, o,
                   bmax, bmax_ld, sel_out, kv_div, static_cast<int>(n_prot), static_cast<int>(sink_end),
                   static_cast<int>(recent_start), static_cast<int>(rec_begin), static_cast<int>(n_rec),
                   static_cast<int>(tokens)};
  if (f16) launch_attn_dt<true>(g, iters, grid, st, a, sel);
  else launch_attn_dt<false>(g, iters, grid, st, a, sel);
  return check_launch(what);
}

}  // namespace

QKV_EXPORT int qkv_sparse_attention(const void* query, const void* key, const void* value,
                                    const int64_t* kv_strides, int64_t batch, int64_t q_heads,
                                    int64_t kv_heads, int64_t tokens, int64_t head_dim,
                                    const int32_t* block_ids, int64_t n_sel, int64_t block,
                                    float scaling, float* workspace, int64_t workspace_bytes,
                                    void* out, int dtype, void* stream) {
  if (!block_ids) return fail(QKV_ERR_INVALID, "qkv_sparse_attention: null pointer");
  return launch_attention("qkv_sparse_attention", query, key, value, kv_strides, batch, q_heads, kv_heads,
                          tokens, head_dim, block_ids, nullptr, 0, nullptr, n_sel, block, scaling, workspace,
                          workspace_bytes, out, dtype, stream);
}

QKV_EXPORT int qkv_sparse_attention_protected(const void* query, const void* key, const void* value,
                                              const int64_t* kv_strides, int64_t batch, int64_t q_heads,
                                              int64_t kv_heads, int64_t history, int64_t head_dim,
                                              const int32_t* block_ids, const float* bmax, int64_t bmax_ld,
                                              int64_t n_sel, int64_t block, int64_t protect_sink,
                                              int64_t protect_recent, int keep_self, float scaling, float* workspace,
                                              int64_t workspace_bytes, int32_t* sel_out, void* out, int dtype,
                                              void* stream) {
  static const char* what = "qkv_sparse_attention_protected";
  if (!block_ids == !bmax) return fail(QKV_ERR_INVALID, "%s: pass exactly one of block_ids and bmax", what);
  if (protect_sink < 0 || protect_recent < 0)
    return fail(QKV_ERR_INVALID, "%s: protected token counts must be >= 0", what);
  return launch_attention(what, query, key, value, kv_strides, batch, q_heads, kv_heads, history, head_dim,
                          block_ids, bmax, bmax_ld, bmax ? sel_out : nullptr, n_sel, block, scaling, workspace,
                          workspace_bytes, out, dtype, stream, 1, protect_sink, protect_recent, keep_self != 0);
}

QKV_EXPORT int qkv_sparse_attention_select(const void* query, const void* key, const void* value,
                                           const int64_t* kv_strides, int64_t batch, int64_t q_heads,
                                           int64_t kv_heads, int64_t tokens, int64_t head_dim,
                                           const float* bmax, int64_t bmax_ld, int64_t n_sel, int64_t block,
                                           float scaling, float* workspace, int64_t workspace_bytes,
                                           int32_t* sel_out, void* out, int dtype, void* stream) {
  if (!bmax) return fail(QKV_ERR_INVALID, "qkv_sparse_attention_select: null pointer");
  return launch_attention("qkv_sparse_attention_select", query, key, value, kv_strides, batch, q_heads,
                          kv_heads, tokens, head_dim, nullptr, bmax, bmax_ld, sel_out, n_sel, block, scaling,
                          workspace, workspace_bytes, out, dtype, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free variant of qkv_sparse_attention_select.  Its workspace
// (row tickets, then per-split partials) is this file-scope device array, one
// copy per GPU, held until the process ends.  Host code never passes the
// array's name to a kernel: the name is a host-side stand-in, and the device
// address of each GPU's copy comes from hipGetSymbolAddress, taken once per
// device with that device current.  Every call on a GPU shares that GPU's
// copy, so calls that overlap in time on one GPU race; the ticket words are
// cleared once per device (by a fill kernel on the caller's stream) and every
// completed call leaves them zero again.
static __device__ __align__(256) float scratch[QKV_NOALLOC_SCRATCH_BYTES / 4];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices];   // device address of `scratch` on each device
bool g_scratch_clear[kMaxDevices];   // ticket words cleared by an eager (uncaptured) fill

__global__ void zero_words_kernel(uint32_t* __restrict__ p, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    p[i] = 0u;
}

}  // namespace

QKV_EXPORT int qkv_sparse_attention_select_noalloc(const void* query, const void* key, const void* value,
                                                   const int64_t* kv_strides, int64_t batch, int64_t q_heads,
                                                   int64_t kv_heads, int64_t tokens, int64_t head_dim,
                                                   const float* bmax, int64_t bmax_ld, int64_t n_sel,
                                                   int64_t block, float scaling, int32_t* sel_out, void* out,
                                                   int dtype, void* stream) {
  static const char* what = "qkv_sparse_attention_select_noalloc";
  if (!bmax) return fail(QKV_ERR_INVALID, "%s: null pointer", what);
  const int64_t need = qkv_sparse_attention_workspace_bytes(batch, q_heads, kv_heads, head_dim, n_sel, block);
  if (need < 0)
    return fail(QKV_ERR_INVALID, "%s: unsupported sizes (head_dim 128, q_heads a multiple of kv_heads, n_sel > 0)",
                what);
  if (need > QKV_NOALLOC_SCRATCH_BYTES)
    return fail(QKV_ERR_UNSUPPORTED, "%s: these sizes need %lld bytes of scratch; the static scratch holds %lld",
                what, (long long)need, (long long)QKV_NOALLOC_SCRATCH_BYTES);
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(QKV_ERR_LAUNCH, "%s: no current device below %d", what, kMaxDevices);
  hipStream_t st = static_cast<hipStream_t>(stream);
  float* ws = nullptr;
  bool clear = false;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
      void* p = nullptr;
      const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p)
        return fail(QKV_ERR_LAUNCH, "%s: hipGetSymbolAddress(scratch) on device %d: %s", what, dev,
                    hipGetErrorString(e));
      g_scratch_ptr[dev] = static_cast<float*>(p);
    }
    ws = g_scratch_ptr[dev];
    clear = g_scratch_clear[dev];
  }
  if (!clear) {
    // Clear the ticket words ahead of the attention kernel on the same
    // stream.  Under graph capture the fill becomes part of the graph (and
    // runs on every replay), so only an eager fill marks the device done.
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess)
      return fail(QKV_ERR_LAUNCH, "%s: hipStreamIsCapturing failed", what);
    zero_words_kernel<<<64, 256, 0, st>>>(reinterpret_cast<uint32_t*>(ws), kTicketWords);
    const int rc = check_launch(what);
    if (rc != QKV_OK) return rc;
    if (cs == hipStreamCaptureStatusNone) {
      std::lock_guard<std::mutex> lock(g_scratch_mu);
      g_scratch_clear[dev] = true;
    }
  }
  return launch_attention(what, query, key, value, kv_strides, batch, q_heads, kv_heads, tokens, head_dim, nullptr,
                          bmax, bmax_ld, sel_out, n_sel, block, scaling, ws, QKV_NOALLOC_SCRATCH_BYTES, out,
                          dtype, stream);
}

QKV_EXPORT int qkv_token_attention(const void* query, const void* key, const void* value,
                                   const int64_t* kv_strides, int64_t batch, int64_t q_heads,
                                   int64_t kv_heads, int64_t tokens, int64_t head_dim,
                                   const int32_t* token_ids, int64_t n_ids, float scaling,
                                   float* workspace, int64_t workspace_bytes, void* out, int dtype,
                                   void* stream) {
  // Every query head is its own row (group size 1) with one-token blocks;
  // row (b, h) reads K/V head h / (q_heads / kv_heads).
  if (!token_ids) return fail(QKV_ERR_INVALID, "qkv_token_attention: null pointer");
  if (kv_heads <= 0 || q_heads % kv_heads)
    return fail(QKV_ERR_INVALID, "qkv_token_attention: q_heads must be a multiple of kv_heads");
  return launch_attention("qkv_token_attention", query, key, value, kv_strides, batch, q_heads, q_heads, tokens,
                          head_dim, token_ids, nullptr, 0, nullptr, n_ids, 1, scaling, workspace, workspace_bytes,
                          out, dtype, stream, static_cast<int>(q_heads / kv_heads));
}
