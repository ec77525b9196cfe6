// Fused relative-position multi-head attention (one kernel per layer).
//
// Replaces the reference's bmmQK -> relShiftB -> add -> softmax -> bmmPV chain
// (src/engines/asr-parakeet/raw-encoder.js:337-344; attention.js:14-138,268-287)
// with one pass that never materialises the [W·H·T, T] score matrix:
//
//   S[i,j] = (q_i + u)·k_j + (q_i + v)·P[c - (i - j)]      (rel_shift closed form:
//            relshift(X)[i,j] = X[i, T-1-i+j], so row T-1-i+j of a [2T-1]-row
//            table; with a table built for Tmax >= T the centre row c = Tmax-1
//            serves every window length, since pe rows depend only on i - j)
//   O_i    = Σ_j softmax_j(S[i,·]) v_j        over keys j < T_w of window w
//
// 1/sqrt(HD) is pre-folded into q, u, v (raw-encoder.js:124-125,133).  Keys past
// a window's length are excluded (key-padding mask), so a window packed with
// others gives the same result as the window alone.
//
// Work decomposition: block = (64-query tile, head, window), 4 waves x 16 query
// rows.  Per 64-key block each wave runs 16 MFMAs for (q+u)kᵀ, 20 for the
// 16x80 band of (q+v)Pᵀ it needs, then an online-softmax update and 16 MFMAs
// for P·V.  The band is turned into the diagonal-shifted score tile through a
// per-wave LDS strip; V is staged transposed in LDS so the P·V B-operand reads
// are 16-byte vectors.
#include "fa_internal.h"
#include "fa_device.h"
#include "attention.h"

#include <type_traits>

namespace fa {

template <typename T>
__device__ __forceinline__ h8 ld8(const T *p) {
  if constexpr (sizeof(T) == 2) {
    return *reinterpret_cast<const h8 *>(p);
  } else {
    const float4 a = reinterpret_cast<const float4 *>(p)[0], b = reinterpret_cast<const float4 *>(p)[1];
    h8 r;
    r[0] = (_Float16)a.x; r[1] = (_Float16)a.y; r[2] = (_Float16)a.z; r[3] = (_Float16)a.w;
    r[4] = (_Float16)b.x; r[5] = (_Float16)b.y; r[6] = (_Float16)b.z; r[7] = (_Float16)b.w;
    return r;
  }
}

template <typename TI, typename TO>
__global__ __launch_bounds__(256) void relpos_attn_kernel(AttnArgs a) {
  constexpr int HD = 128, QB = 64, KB = 64, SW = 80 + 4, PBS = KB + 8, VTS = KB + 8;
  __shared__ __attribute__((aligned(16))) _Float16 sVt[HD * VTS];
  __shared__ float sStrip[4][16 * SW];
  __shared__ __attribute__((aligned(16))) _Float16 sP[4][16 * PBS];

  const int w = blockIdx.z, h = blockIdx.y, qb = blockIdx.x;
  const int T = a.win.len[w], off = a.win.off[w];
  if (qb * QB >= T) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c16 = lane & 15;
  const int i0 = qb * QB + wave * 16;  // this wave's first query (window-local)
  const TI *Q = reinterpret_cast<const TI *>(a.q) + (size_t)off * a.ldq + h * HD;
  const TI *Kp = reinterpret_cast<const TI *>(a.k) + (size_t)off * a.ldk + h * HD;
  const TI *Vp = reinterpret_cast<const TI *>(a.v) + (size_t)off * a.ldv + h * HD;
  const TI *Pp = reinterpret_cast<const TI *>(a.pos) + h * HD;

  // A operands: (q+u) and (q+v) for row i0 + c16, d = s*32 + g*8 .. +8
  h8 qu[4], qv[4];
  {
    const int qi = min(i0 + c16, T - 1);
    const TI *qr = Q + (size_t)qi * a.ldq;
#pragma unroll
    for (int s = 0; s < 4; s++) {
      const int d = s * 32 + g * 8;
      h8 x = ld8(qr + d);
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float xv = (float)x[e];
        qu[s][e] = (_Float16)(xv + a.pbu[h * HD + d + e]);
        qv[s][e] = (_Float16)(xv + a.pbv[h * HD + d + e]);
      }
    }
  }

  f4 o[8];
#pragma unroll
  for (int t = 0; t < 8; t++) o[t] = f4{0.f, 0.f, 0.f, 0.f};
  float mrow[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY}, lrow[4] = {0.f, 0.f, 0.f, 0.f};
  float *strip = sStrip[wave];
  _Float16 *pb = sP[wave];

  for (int j0 = 0; j0 < T; j0 += KB) {
    // stage V[j0 .. j0+64) transposed: sVt[d][key]
    __syncthreads();
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const int idx = tid + c * 256, key = idx >> 4, dc = (idx & 15) * 8;
      const int kj = min(j0 + key, T - 1);
      h8 x = ld8(Vp + (size_t)kj * a.ldv + dc);
#pragma unroll
      for (int e = 0; e < 8; e++) sVt[(dc + e) * VTS + key] = x[e];
    }

    // content scores (q+u)·kᵀ : 4 tiles of 16 keys
    f4 sc[4];
#pragma unroll
    for (int jt = 0; jt < 4; jt++) {
      sc[jt] = f4{0.f, 0.f, 0.f, 0.f};
      const int kj = min(j0 + jt * 16 + c16, T - 1);
      const TI *kr = Kp + (size_t)kj * a.ldk;
#pragma unroll
      for (int s = 0; s < 4; s++) sc[jt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qu[s], ld8(kr + s * 32 + g * 8), sc[jt], 0, 0, 0);
    }
    // positional band (q+v)·Pᵀ over table rows pr0 .. pr0+79
    const int pr0 = a.pcenter - (i0 + 15) + j0;
#pragma unroll
    for (int ct = 0; ct < 5; ct++) {
      f4 bd = f4{0.f, 0.f, 0.f, 0.f};
      const int pr = min(max(pr0 + ct * 16 + c16, 0), a.prows - 1);
      const TI *prow = Pp + (size_t)pr * a.ldp;
#pragma unroll
      for (int s = 0; s < 4; s++) bd = __builtin_amdgcn_mfma_f32_16x16x32_f16(qv[s], ld8(prow + s * 32 + g * 8), bd, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; r++) strip[(g * 4 + r) * SW + ct * 16 + c16] = bd[r];
    }
    __syncthreads();  // strip visible to the wave's lanes; sVt complete
    // S = ac + band[i][j - j0 + 15 - (i - i0)], mask keys >= T, online softmax
    float mnew[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int ri = g * 4 + r;
      float mx = mrow[r];
#pragma unroll
      for (int jt = 0; jt < 4; jt++) {
        const int jj = jt * 16 + c16;
        float v = sc[jt][r] + strip[ri * SW + jj + 15 - ri];
        v = (j0 + jj < T) ? v : -INFINITY;
        sc[jt][r] = v;
        mx = fmaxf(mx, v);
      }
      mnew[r] = row16_max(mx);
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const float corr = __expf(mrow[r] - mnew[r]);
      float ls = 0.f;
#pragma unroll
      for (int jt = 0; jt < 4; jt++) {
        const float pv = __expf(sc[jt][r] - mnew[r]);
        ls += pv;
        pb[(g * 4 + r) * PBS + jt * 16 + c16] = (_Float16)pv;
      }
      lrow[r] = lrow[r] * corr + row16_sum(ls);
      mrow[r] = mnew[r];
#pragma unroll
      for (int t = 0; t < 8; t++) o[t][r] *= corr;
    }
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    // O += P·V
#pragma unroll
    for (int kk = 0; kk < 2; kk++) {
      const h8 pa = *reinterpret_cast<const h8 *>(&pb[c16 * PBS + kk * 32 + g * 8]);
#pragma unroll
      for (int t = 0; t < 8; t++) {
        const h8 vb = *reinterpret_cast<const h8 *>(&sVt[(t * 16 + c16) * VTS + kk * 32 + g * 8]);
        o[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, vb, o[t], 0, 0, 0);
      }
    }
  }

  TO *O = reinterpret_cast<TO *>(a.out) + (size_t)off * a.ldo + h * HD;
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int i = i0 + g * 4 + r;
    if (i >= T) continue;
    const float inv = 1.f / lrow[r];
#pragma unroll
    for (int t = 0; t < 8; t++) O[(size_t)i * a.ldo + t * 16 + c16] = (TO)(o[t][r] * inv);
  }
}

// ── f16 encoder attention: LDS-staged, direct-to-LDS copies ────────────────
// Same math as relpos_attn_kernel, for the fused encoder's f16 q|k|v buffer.
// Per 64-key block the workgroup copies its K tile [64][128], the
// transposed V tile [128 d][64 keys] (from v_transpose_kernel's buffer) and
// the union of its four waves' positional bands [128 rows][128] into LDS with
// global_load_lds_dwordx4, two blocks in flight; every MFMA operand is then a
// 16-byte LDS read.  Rows are XOR-swizzled in 16-byte chunks (chunk ^ (row & 7))
// so the 8 rows one ds_read_b128 phase touches hit distinct banks.

// Vt[w][h][d][Tp] = V[off_w + t][h*HD + d] for t < T_w, 0 for T_w <= t < Tp.
__global__ __launch_bounds__(256) void v_transpose_kernel(const _Float16 *__restrict__ v, int ldv, WinTable win, int H, int Tp,
                                                          _Float16 *__restrict__ vt) {
  constexpr int HD = 128, TS = 64;
  __shared__ _Float16 tile[TS][HD + 8];
  const int t0 = blockIdx.x * TS, h = blockIdx.y, w = blockIdx.z, tid = threadIdx.x;
  if (t0 >= Tp) return;
  const int T = win.len[w];
  const _Float16 *src = v + (size_t)win.off[w] * ldv + h * HD;
#pragma unroll
  for (int c = 0; c < 4; c++) {  // 64 rows x 16 chunks of 8 halfs
    const int idx = tid + c * 256, r = idx >> 4, ch = idx & 15;
    h8 x = h8{0, 0, 0, 0, 0, 0, 0, 0};
    if (t0 + r < T) x = *reinterpret_cast<const h8 *>(src + (size_t)(t0 + r) * ldv + ch * 8);
    *reinterpret_cast<h8 *>(&tile[r][ch * 8]) = x;
  }
  __syncthreads();
  _Float16 *dst = vt + ((size_t)(w * H + h) * HD) * Tp + t0;
#pragma unroll
  for (int c = 0; c < 4; c++) {  // 128 d rows x 8 chunks of 8 keys
    const int idx = tid + c * 256, d = idx >> 3, ch = idx & 7;
    h8 x;
#pragma unroll
    for (int e = 0; e < 8; e++) x[e] = tile[ch * 8 + e][d];
    *reinterpret_cast<h8 *>(dst + (size_t)d * Tp + ch * 8) = x;
  }
}

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// global -> LDS, 16 B per lane (lane i lands at lds_addr + 16 i); M0 carries the
// wave-uniform LDS address.  Completion is tracked with explicit vmcnt waits.
__device__ __forceinline__ void attn_dma16(const void *g, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds_addr) : "memory", "m0");
}
// the same copy from a wave-uniform base (SGPRs) plus the lane's 32-bit byte
// offset: a block's copies then change only the scalar base
__device__ __forceinline__ void attn_dma16_s(uint32_t voff, const void *sbase, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds_addr) : "memory", "m0");
}
#pragma clang diagnostic pop

// Workgroup = QB = 16·NWV queries of one (window, head), one 16-query row
// tile per wave: every product is computed with keys / band rows as
// the MFMA's M side and the wave's 16 queries as N, so each lane owns ONE
// query (column c16) and the softmax state (reference max, partial sum,
// rescale factor) is per lane.  Keys advance 32 per block; S blocks of
// copies are in flight (global_load_lds_dwordx4, tracked with vmcnt):
//   K   [32 keys][128 d]   (256 B rows, 16-byte chunk c at slot c ^ ((row >> 1) & 7):
//                           the 8 rows 2 m + kt one read phase touches hit distinct banks)
//   Vt  [128 d][32 keys]   (64 B rows,  chunk c at slot c ^ ((row >> 1) & 3))
// The positional band of a key block is table rows pbase0 + j0 + [0, BR),
// BR = QB + 32 (query i and key j use band row (j - j0) + (q0 + QB - 1 - i)).
// Consecutive blocks' bands overlap in BR - 32 rows, so the band lives in a
// ring of RS table rows (row x at slot x % RS, chunk c at c ^ (slot & 7)):
// the first block copies its BR rows, every later block only the 32 it adds.
//   * Key tile kt (0, 1) of a 32-key block reads K rows 2 m + kt for MFMA row
//     m, so output row g*4 + r of tile kt is key 8 g + 2 r + kt: lane (g, c16)
//     holds keys 8 g .. 8 g + 7 of its query, in order.  Its probabilities
//     are then directly the B operand of O^T += Vt · P^T (B[k][n], k = 8 g ..
//     8 g + 7): no LDS round trip for P.
//   * The positional band is computed as band^T (rows = table rows, columns =
//     queries) and stored per query column, 4 rows per ds_write_b128; the key
//     (r, kt) of lane (g, c16) uses band offset 8 g + 15 - c16 + 2 r + kt:
//     8 consecutive floats of the lane's own column.
//   * Scores are carried in log2 units (scaled by log2 e once summed), so a
//     probability is one v_exp_f32.
//   * Keys are masked only in blocks that reach past the window or when the
//     attention is chunk-limited (per-lane key range computed once).
template <int NWV, int S>
__global__ __launch_bounds__(64 * NWV) __attribute__((amdgpu_waves_per_eu((NWV + 3) / 4, (NWV + 3) / 4))) void relpos_attn_t_kernel(
    AttnArgs a, const _Float16 *__restrict__ vt, int Tp) {
  constexpr int HD = 128, QB = 16 * NWV, KB = 32, BR = QB + 32;
  constexpr int RS = BR + (S - 1) * KB <= 128 ? 128 : 256;  // band ring rows (power of two)
  static_assert(BR + (S - 1) * KB <= RS, "band ring holds the current band and the prefetched blocks' rows");
  constexpr int IT0 = 16 + BR / 4, IT1 = 16 + KB / 4;
  constexpr int IW0 = (IT0 + NWV - 1) / NWV, IW1 = (IT1 + NWV - 1) / NWV;
  static_assert(IT1 % NWV == 0, "equal copy counts per wave (vmcnt accounting)");
  constexpr int KBYTES = KB * 256, VBYTES = HD * 64, KVB = KBYTES + VBYTES;
  constexpr int SW = 48 + 4;  // band strip: [16 query columns][SW floats]
  constexpr float L2E = 1.4426950408889634f, kLazy = 11.f;  // lazy rescale threshold (log2 units)
  __shared__ __attribute__((aligned(1024))) char kvs[S][KVB];
  __shared__ __attribute__((aligned(1024))) char ring[RS * 256];
  __shared__ __attribute__((aligned(16))) float sStrip[NWV][16 * SW];

  const int w = blockIdx.z, h = blockIdx.y, q0 = blockIdx.x * QB;
  const int T = a.win.len[w], off = a.win.off[w];
  if (q0 >= T) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, c16 = lane & 15;
  const int iw = q0 + wave * 16;  // this wave's first query (window-local)
  const int qi = iw + c16;        // this lane's query
  const _Float16 *Q = reinterpret_cast<const _Float16 *>(a.q) + (size_t)off * a.ldq + h * HD;
  const _Float16 *Kp = reinterpret_cast<const _Float16 *>(a.k) + (size_t)off * a.ldk + h * HD;
  const _Float16 *Pp = reinterpret_cast<const _Float16 *>(a.pos) + h * HD;
  const _Float16 *Vt = vt + ((size_t)(w * a.H + h) * HD) * Tp;
  const uint32_t sadr0 = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) char *)kvs[0]);
  const uint32_t radr = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) char *)ring);
  const int pbase0 = a.pcenter - (q0 + QB - 1);

  // LDS layouts (64 banks read 16 lanes = 256 bytes at a time): a 256-byte K
  // or band row r keeps its 16-byte chunk c at slot c ^ (key / band row & 15),
  // a 64-byte Vt row d its chunk c at slot c ^ ((d >> 2) & 3), so the 16 rows
  // one read phase touches hit distinct banks.
  // copy i of this wave: the lane's byte offset from the block's scalar base
  // (K rows, Vt rows, band rows), the same for every block
  uint32_t voff[IW0];
#pragma unroll
  for (int i = 0; i < IW0; i++) {
    const int ins = wave + i * NWV;
    if (ins < 8) {
      const int r = ins * 4 + (lane >> 4), ch = (lane & 15) ^ ((r >> 1) & 15);
      voff[i] = (uint32_t)(r * a.ldk + ch * 8) * 2;
    } else if (ins < 16) {
      const int r = (ins - 8) * 16 + (lane >> 2), ch = (lane & 3) ^ ((r >> 2) & 3);
      voff[i] = (uint32_t)(r * Tp + ch * 8) * 2;
    } else {
      const int rl = (ins - 16) * 4 + (lane >> 4), ch = (lane & 15) ^ (rl & 15);
      voff[i] = (uint32_t)(rl * a.ldp + ch * 8) * 2;
    }
  }
  auto issue = [&](int sidx, int j0, int rb, auto first) {
    constexpr bool F = decltype(first)::value;
    constexpr int IT = F ? IT0 : IT1, IW = F ? IW0 : IW1, R0 = F ? 0 : BR - KB, PN = F ? BR : KB;
    const uint32_t base = sadr0 + (uint32_t)sidx * KVB;
    // rows past the window (keys) or outside the positional table (band) are
    // clamped, in the blocks that have them, with per-lane addresses
    const bool kclamp = j0 + KB > T;
    const int prow0 = pbase0 + j0 + R0;  // the first band row this issue copies (rb + R0 is a multiple of 16)
    const bool pclamp = prow0 < 0 || prow0 + PN > a.prows;
#pragma unroll
    for (int i = 0; i < IW; i++) {
      const int ins = wave + i * NWV;
      if (IT % NWV != 0 && ins >= IT) break;
      if (ins < 8) {
        const uint32_t dst = base + ins * 1024;
        if (!kclamp) {
          attn_dma16_s(voff[i], Kp + (size_t)j0 * a.ldk, dst);
        } else {
          const int r = ins * 4 + (lane >> 4), ch = (lane & 15) ^ ((r >> 1) & 15);
          attn_dma16(Kp + (size_t)min(j0 + r, T - 1) * a.ldk + ch * 8, dst);
        }
      } else if (ins < 16) {
        attn_dma16_s(voff[i], Vt + j0, base + ins * 1024);
      } else {
        const int x = rb + R0 + (ins - 16) * 4;
        const uint32_t dst = radr + (uint32_t)(x & (RS - 1)) * 256;
        if (!pclamp) {
          attn_dma16_s(voff[i], Pp + (size_t)prow0 * a.ldp, dst);
        } else {
          const int rl = (ins - 16) * 4 + (lane >> 4), ch = (lane & 15) ^ (rl & 15);
          const int pr = min(max(prow0 + rl, 0), a.prows - 1);
          attn_dma16(Pp + (size_t)pr * a.ldp + ch * 8, dst);
        }
      }
    }
  };

  // keys this lane's query sees, and the key blocks the workgroup needs
  int klo = 0, khi = T - 1, jlo = 0, jhi = T;
  if (a.chunk > 0) {
    const int cs = a.chunk * (qi / a.chunk);
    klo = max(0, cs - a.left);
    khi = min(T - 1, cs + a.chunk - 1 + a.right);
    const int qlast = min(T, q0 + QB) - 1;
    jlo = max(0, a.chunk * (q0 / a.chunk) - a.left);
    jhi = min(T, a.chunk * (qlast / a.chunk) + a.chunk + a.right);
  }
  const int kb0 = jlo / KB, nkb = (jhi + KB - 1) / KB;
  issue(0, kb0 * KB, 0, std::true_type{});
#pragma unroll
  for (int p = 1; p < S - 1; p++)
    if (kb0 + p < nkb) issue(p, (kb0 + p) * KB, p * KB, std::false_type{});

  // the first blocks' copies are in flight while q is loaded and biased
  // B operands: (q+u) and (q+v) of this lane's query, d = s*32 + g*8 .. +8
  h8 qu[4], qv[4];
  {
    const _Float16 *qr = Q + (size_t)min(qi, T - 1) * a.ldq;
#pragma unroll
    for (int s = 0; s < 4; s++) {
      const int d = s * 32 + g * 8;
      const h8 x = *reinterpret_cast<const h8 *>(qr + d);
      const float4 *bu = reinterpret_cast<const float4 *>(a.pbu + h * HD + d), *bv = reinterpret_cast<const float4 *>(a.pbv + h * HD + d);
      const float4 u0 = bu[0], u1 = bu[1], v0 = bv[0], v1 = bv[1];
      const float ub[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w}, vb[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float xv = (float)x[e];
        qu[s][e] = (_Float16)(xv + ub[e]);
        qv[s][e] = (_Float16)(xv + vb[e]);
      }
    }
  }

  f4 o[8];  // O^T tiles: d rows t*16 + g*4 + r, query column c16
#pragma unroll
  for (int t = 0; t < 8; t++) o[t] = f4{0.f, 0.f, 0.f, 0.f};
  float mref = -INFINITY, lpart = 0.f;
  const int lbw = QB - 16 - wave * 16;  // band offset of this wave's union tile 0
  float *strip = sStrip[wave];

  for (int kb = kb0; kb < nkb; kb++) {
    const int j0 = kb * KB, cur = (kb - kb0) % S;
    // this block's copies landed: at most min(S - 2, blocks after it) later blocks' copies outstanding
    const int ahead = min(S - 2, nkb - 1 - kb);
    if (S > 2 && ahead >= 2) __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8) | (((2 * IW1) & 15) | (((2 * IW1) >> 4) << 14)));
    else if (S > 2 && ahead == 1) __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8) | ((IW1 & 15) | ((IW1 >> 4) << 14)));
    else __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
    __syncthreads();
    const int rb = (kb - kb0) * KB;
    if (kb + S - 1 < nkb) issue((cur + S - 1) % S, j0 + (S - 1) * KB, rb + (S - 1) * KB, std::false_type{});
    const char *Ks = kvs[cur], *Vs = Ks + KBYTES;

    h8 kf[2][4], pf[3][4];
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
      const int r = 2 * c16 + kt;  // MFMA row c16 of key tile kt = key 2 c16 + kt
#pragma unroll
      for (int s = 0; s < 4; s++) kf[kt][s] = *reinterpret_cast<const h8 *>(Ks + r * 256 + (((s * 4 + g) ^ ((r >> 1) & 15)) * 16));
    }
#pragma unroll
    for (int u = 0; u < 3; u++) {
      const int sl = (rb + lbw + u * 16 + c16) & (RS - 1);
#pragma unroll
      for (int s = 0; s < 4; s++) pf[u][s] = *reinterpret_cast<const h8 *>(ring + sl * 256 + (((s * 4 + g) ^ (sl & 15)) * 16));
    }
    __builtin_amdgcn_sched_barrier(0);
    f4 sc[2], bd[3];
#pragma unroll
    for (int kt = 0; kt < 2; kt++) sc[kt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < 3; u++) bd[u] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; s++) {
#pragma unroll
      for (int kt = 0; kt < 2; kt++) sc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[kt][s], qu[s], sc[kt], 0, 0, 0);
#pragma unroll
      for (int u = 0; u < 3; u++) bd[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pf[u][s], qv[s], bd[u], 0, 0, 0);
    }
    // Vt fragments (d rows t*16 + c16, keys g*8 .. +8), read now to hide behind the softmax
    h8 vf[8];
#pragma unroll
    for (int t = 0; t < 8; t++) {
      const int d = t * 16 + c16;
      vf[t] = *reinterpret_cast<const h8 *>(Vs + d * 64 + ((g ^ ((d >> 2) & 3)) * 16));
    }
#pragma unroll
    for (int u = 0; u < 3; u++) *reinterpret_cast<f4 *>(strip + c16 * SW + u * 16 + g * 4) = bd[u];
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): strip written (wave-private)
    __builtin_amdgcn_wave_barrier();
    float sv[8];  // keys 8 g + e of this lane's query (e = 2 r + kt)
    {
      const float *bp = strip + c16 * SW + 8 * g + 15 - c16;
#pragma unroll
      for (int r = 0; r < 4; r++)
#pragma unroll
        for (int kt = 0; kt < 2; kt++) sv[2 * r + kt] = (sc[kt][r] + bp[2 * r + kt]) * L2E;
    }
    if (j0 + KB > T || a.chunk > 0) {
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const int j = j0 + 8 * g + e;
        sv[e] = (j >= klo && j <= khi) ? sv[e] : -INFINITY;
      }
    }
    float mx = sv[0];
#pragma unroll
    for (int e = 1; e < 8; e++) mx = fmaxf(mx, sv[e]);
    if (__builtin_amdgcn_ballot_w64(mx > mref + kLazy)) {
      // new reference max for every query whose running max moved: the
      // query's 4 lane groups agree through the xor-16 / xor-32 exchange
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      if (mx > mref) {
        const float corr = __builtin_amdgcn_exp2f(mref - mx);  // 0 on the first visible block (mref = -inf)
        lpart *= corr;
#pragma unroll
        for (int t = 0; t < 8; t++) o[t] *= corr;
        mref = mx;
      }
    }
    h8 pb;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      // masked keys give 0 (also while the query has seen no visible key: -inf - -inf)
      const float p = sv[e] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(sv[e] - mref);
      lpart += p;
      pb[e] = (_Float16)p;
    }
#pragma unroll
    for (int t = 0; t < 8; t++) o[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[t], pb, o[t], 0, 0, 0);
  }

  float lsum = lpart + __shfl_xor(lpart, 16);
  lsum += __shfl_xor(lsum, 32);
  if (qi >= T) return;
  const float inv = 1.f / lsum;
  _Float16 *O = reinterpret_cast<_Float16 *>(a.out) + (size_t)(off + qi) * a.ldo + h * HD + g * 4;
  _Float16 *Olo = a.out_lo ? reinterpret_cast<_Float16 *>(a.out_lo) + (size_t)(off + qi) * a.ldo + h * HD + g * 4 : nullptr;
#pragma unroll
  for (int t = 0; t < 8; t++) {
    h4 hi, lo;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const float v = o[t][r] * inv;
      hi[r] = (_Float16)v;
      lo[r] = (_Float16)(v - (float)hi[r]);
    }
    *reinterpret_cast<h4 *>(O + t * 16) = hi;
    if (Olo) *reinterpret_cast<h4 *>(Olo + t * 16) = lo;
  }
}

int relpos_attention_f16(fa_ctx *ctx, const AttnArgs &a, int Tmax, _Float16 *vt, const char *label, bool transpose) {
  const int W = a.win.n;
  if (a.HD != 128) return set_err(ctx, FA_E_UNSUPPORTED, "%s: head dim %d (kernel is specialised for 128)", label, a.HD);
  if (Tmax <= 0 || W <= 0) return FA_OK;
  if (W > kMaxWin) return set_err(ctx, FA_E_INVALID, "%s: %d windows in one launch (max %d)", label, W, kMaxWin);
  for (int i = 0; i < W; i++)
    if (a.win.len[i] > Tmax || a.pcenter - (a.win.len[i] - 1) < 0 || a.pcenter + a.win.len[i] - 1 >= a.prows)
      return set_err(ctx, FA_E_INVALID, "%s: window %d length %d outside the positional table", label, i, a.win.len[i]);
  const int Tp = (Tmax + 63) / 64 * 64;  // v_transpose_kernel tiles of 64 keys; the attention reads 32 at a time
  if (transpose) {
    ProfScope ps(ctx, "v_transpose");
    FA_LAUNCH(ps, v_transpose_kernel, dim3(Tp / 64, a.H, W), dim3(256), 0, ctx->stream, reinterpret_cast<const _Float16 *>(a.v), a.ldv, a.win, a.H,
              Tp, vt);
    FA_TRY(check_launch(ctx, "v_transpose"));
  }
  ProfScope ps(ctx, label);
  // 96-query workgroups (6 waves, 1.5 per SIMD; a 188-frame window splits
  // 96 + 92), K / Vt / band copies one block ahead
  FA_LAUNCH(ps, (relpos_attn_t_kernel<6, 2>), dim3(cdiv(Tmax, 96), a.H, W), dim3(384), 0, ctx->stream, a, (const _Float16 *)vt, Tp);
  return check_launch(ctx, label);
}

int relpos_attention(fa_ctx *ctx, const AttnArgs &a, int in_f32, int out_f32, int Tmax, const char *label) {
  const int W = a.win.n;
  if (a.HD != 128) return set_err(ctx, FA_E_UNSUPPORTED, "%s: head dim %d (kernel is specialised for 128)", label, a.HD);
  if (Tmax <= 0 || W <= 0) return FA_OK;
  if (W > kMaxWin) return set_err(ctx, FA_E_INVALID, "%s: %d windows in one launch (max %d)", label, W, kMaxWin);
  dim3 grid(cdiv(Tmax, 64), a.H, W);
  ProfScope ps(ctx, label);
  if (!in_f32 && !out_f32)
    FA_LAUNCH(ps, (relpos_attn_kernel<_Float16, _Float16>), grid, dim3(256), 0, ctx->stream, a);
  else if (in_f32 && out_f32)
    FA_LAUNCH(ps, (relpos_attn_kernel<float, float>), grid, dim3(256), 0, ctx->stream, a);
  else
    return set_err(ctx, FA_E_UNSUPPORTED, "%s: mixed attention I/O types", label);
  return check_launch(ctx, label);
}

}  // namespace fa

