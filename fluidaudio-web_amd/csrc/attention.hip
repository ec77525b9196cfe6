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
#pragma clang diagnostic pop

// Workgroup = QB = 16·RT·NWV queries of one (window, head): NWV waves, each
// owning RT 16-row MFMA tiles (with RT = 2 every K / V / band fragment read
// from LDS feeds two MFMAs; with RT = 1 more waves share a CU).  Keys advance
// 32 per stage, two stages in flight:
//   K   [32 keys][128 d]        (256 B rows, 16-byte chunk c at slot c ^ (row & 7))
//   Vt  [128 d][32 keys]        (64 B rows,  chunk c at slot c ^ ((row >> 1) & 3))
//   band [QB+32 rows][128 d]    table rows pbase .. , pbase = pc - (q0 + QB - 1) + j0
// A query i and key j use band row (j - j0) + (q0 + QB - 1 - i).
template <int RT, int NWV>
__global__ __launch_bounds__(64 * NWV) __attribute__((amdgpu_waves_per_eu(NWV > 4 ? 2 : 1, NWV > 4 ? 2 : 1))) void relpos_attn_lds_kernel(
    AttnArgs a, const _Float16 *__restrict__ vt, int Tp) {
  constexpr int HD = 128, QB = 16 * RT * NWV, KB = 32, BR = QB + 32, UT = RT + 2;  // UT: band tiles per wave
  constexpr int IT = 16 + BR / 4, IW = IT / NWV;                                  // 1 KB copies per stage / per wave
  static_assert(IT % NWV == 0, "copies per wave");
  constexpr int KBYTES = KB * 256, VBYTES = HD * 64, PBYTES = BR * 256;
  constexpr int STG = KBYTES + VBYTES + PBYTES;  // 56 KB
  constexpr int SW = 48 + 4, PBS = KB + 8;         // strip row stride (floats), probability row stride (halfs)
  __shared__ __attribute__((aligned(1024))) char st0[STG];
  __shared__ __attribute__((aligned(1024))) char st1[STG];
  __shared__ float sStrip[NWV][RT][16 * SW];
  __shared__ __attribute__((aligned(16))) _Float16 sP[NWV][RT][16 * PBS];

  const int w = blockIdx.z, h = blockIdx.y, q0 = blockIdx.x * QB;
  const int T = a.win.len[w], off = a.win.off[w];
  if (q0 >= T) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, c16 = lane & 15;
  const int iw = q0 + wave * 16 * RT;  // this wave's first query (window-local); row tile rt covers iw + 16 rt ..
  const _Float16 *Q = reinterpret_cast<const _Float16 *>(a.q) + (size_t)off * a.ldq + h * HD;
  const _Float16 *Kp = reinterpret_cast<const _Float16 *>(a.k) + (size_t)off * a.ldk + h * HD;
  const _Float16 *Pp = reinterpret_cast<const _Float16 *>(a.pos) + h * HD;
  const _Float16 *Vt = vt + ((size_t)(w * a.H + h) * HD) * Tp;
  const uint32_t sadr[2] = {(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) char *)st0),
                            (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) char *)st1)};
  const int pbase0 = a.pcenter - (q0 + QB - 1);

  // 56 copies of 1 KB per stage, 14 per wave: K (8: 4 rows each), Vt (8: 16
  // rows each), band (40: 4 rows each).
  auto issue = [&](int sidx, int j0) {
    const uint32_t base = sadr[sidx];
#pragma unroll
    for (int i = 0; i < IW; i++) {
      const int ins = wave + i * NWV;  // 0..IT-1
      const void *src;
      if (ins < 8) {
        const int r = ins * 4 + (lane >> 4), ch = (lane & 15) ^ (r & 7);
        src = Kp + (size_t)min(j0 + r, T - 1) * a.ldk + ch * 8;
      } else if (ins < 16) {
        const int r = (ins - 8) * 16 + (lane >> 2), ch = (lane & 3) ^ ((r >> 1) & 3);
        src = Vt + (size_t)r * Tp + j0 + ch * 8;
      } else {
        const int r = (ins - 16) * 4 + (lane >> 4), ch = (lane & 15) ^ (r & 7);
        const int pr = min(max(pbase0 + j0 + r, 0), a.prows - 1);
        src = Pp + (size_t)pr * a.ldp + ch * 8;
      }
      attn_dma16(src, base + ins * 1024);
    }
  };

  // A operands: (q+u) and (q+v) for rows iw + 16 rt + c16, d = s*32 + g*8 .. +8
  h8 qu[RT][4], qv[RT][4];
#pragma unroll
  for (int rt = 0; rt < RT; rt++) {
    const int qi = min(iw + rt * 16 + c16, T - 1);
    const _Float16 *qr = Q + (size_t)qi * a.ldq;
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
        qu[rt][s][e] = (_Float16)(xv + ub[e]);
        qv[rt][s][e] = (_Float16)(xv + vb[e]);
      }
    }
  }
  // key blocks this workgroup's queries can see (all keys, or the union of
  // their chunk windows when attention is chunk-limited)
  int jlo = 0, jhi = T;
  if (a.chunk > 0) {
    const int qlast = min(T, q0 + QB) - 1;
    jlo = max(0, a.chunk * (q0 / a.chunk) - a.left);
    jhi = min(T, a.chunk * (qlast / a.chunk) + a.chunk + a.right);
  }
  const int kb0 = jlo / KB, nkb = (jhi + KB - 1) / KB;
  issue(0, kb0 * KB);

  f4 o[RT][8];
#pragma unroll
  for (int rt = 0; rt < RT; rt++)
#pragma unroll
    for (int t = 0; t < 8; t++) o[rt][t] = f4{0.f, 0.f, 0.f, 0.f};
  float mrow[RT][4], lrow[RT][4];
#pragma unroll
  for (int rt = 0; rt < RT; rt++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      mrow[rt][r] = -INFINITY;
      lrow[rt][r] = 0.f;
    }
  const int lbw = QB - 16 * RT - wave * 16 * RT;  // band row of this wave's union tile 0 (= the last row tile's first band row)

  for (int kb = kb0; kb < nkb; kb++) {
    const int j0 = kb * KB, cur = (kb - kb0) & 1;
    __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));  // vmcnt(0): this stage's copies landed
    __syncthreads();                                    // ... for every wave; the other stage is free
    if (kb + 1 < nkb) issue(cur ^ 1, j0 + KB);
    const char *Ks = cur ? st1 : st0, *Vs = Ks + KBYTES, *Ps = Ks + KBYTES + VBYTES;

    // fragment reads: K (2 key tiles x 4 k-steps), band (4 union tiles x 4)
    h8 kf[2][4], pf[UT][4];
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
      const int r = kt * 16 + c16;
#pragma unroll
      for (int s = 0; s < 4; s++) kf[kt][s] = *reinterpret_cast<const h8 *>(Ks + r * 256 + (((s * 4 + g) ^ (r & 7)) * 16));
    }
#pragma unroll
    for (int u = 0; u < UT; u++) {
      const int r = lbw + u * 16 + c16;
#pragma unroll
      for (int s = 0; s < 4; s++) pf[u][s] = *reinterpret_cast<const h8 *>(Ps + r * 256 + (((s * 4 + g) ^ (r & 7)) * 16));
    }
    __builtin_amdgcn_sched_barrier(0);
    // row tile rt uses band union tiles (RT - 1 - rt) .. (RT + 1 - rt)
    f4 sc[RT][2], bd[RT][3];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
#pragma unroll
      for (int kt = 0; kt < 2; kt++) sc[rt][kt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ct = 0; ct < 3; ct++) bd[rt][ct] = f4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int s = 0; s < 4; s++)
#pragma unroll
      for (int rt = 0; rt < RT; rt++) {
#pragma unroll
        for (int kt = 0; kt < 2; kt++) sc[rt][kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qu[rt][s], kf[kt][s], sc[rt][kt], 0, 0, 0);
#pragma unroll
        for (int ct = 0; ct < 3; ct++) bd[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qv[rt][s], pf[RT - 1 - rt + ct][s], bd[rt][ct], 0, 0, 0);
      }
    // V fragments (d rows t*16 + c16, keys g*8 .. +8), read now to hide behind the softmax
    h8 vf[8];
#pragma unroll
    for (int t = 0; t < 8; t++) {
      const int d = t * 16 + c16;
      vf[t] = *reinterpret_cast<const h8 *>(Vs + d * 64 + ((g ^ ((d >> 1) & 3)) * 16));
    }
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
      for (int ct = 0; ct < 3; ct++)
#pragma unroll
        for (int rr = 0; rr < 4; rr++) sStrip[wave][rt][(g * 4 + rr) * SW + ct * 16 + c16] = bd[rt][ct][rr];
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): strip writes done (wave-private strips)
    __builtin_amdgcn_wave_barrier();
    // S = ac + band[i][jj + 15 - (i - ib)], keys >= T masked, online softmax.
    // Lazy rescaling: probabilities are taken against a per-row reference
    // max mref that only moves (rescaling l and O) when some row's running
    // max exceeds it by more than kLazy nats, decided wave-wide; p <= e^kLazy
    // stays well inside f16 range with unchanged relative precision.
    constexpr float kLazy = 8.f;
    float sv[RT][4][2];
    bool need = false;
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
      const float *strip = sStrip[wave][rt];
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int ri = g * 4 + r;
        float v0 = sc[rt][0][r] + strip[ri * SW + c16 + 15 - ri];
        float v1 = sc[rt][1][r] + strip[ri * SW + 16 + c16 + 15 - ri];
        int klo = 0, khi = T - 1;  // keys this query sees
        if (a.chunk > 0) {
          const int i = iw + rt * 16 + ri, cs = a.chunk * (i / a.chunk);
          klo = max(klo, cs - a.left);
          khi = min(khi, cs + a.chunk - 1 + a.right);
        }
        v0 = (j0 + c16 >= klo && j0 + c16 <= khi) ? v0 : -INFINITY;
        v1 = (j0 + 16 + c16 >= klo && j0 + 16 + c16 <= khi) ? v1 : -INFINITY;
        sv[rt][r][0] = v0;
        sv[rt][r][1] = v1;
        need |= fmaxf(v0, v1) > mrow[rt][r] + kLazy;
      }
    }
    if (__builtin_amdgcn_ballot_w64(need)) {
#pragma unroll
      for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const float mx = row16_max(fmaxf(sv[rt][r][0], sv[rt][r][1]));
          if (mx > mrow[rt][r]) {
            const float corr = __expf(mrow[rt][r] - mx);  // 0 on the first key block (mref = -inf)
            lrow[rt][r] *= corr;  // per-lane partial sums scale with their row
#pragma unroll
            for (int t = 0; t < 8; t++) o[rt][t][r] *= corr;
            mrow[rt][r] = mx;
          }
        }
    }
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
      _Float16 *pb = sP[wave][rt];
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int ri = g * 4 + r;
        // masked keys give 0 (also while a row has seen no visible key yet: -inf - -inf)
        const float p0 = sv[rt][r][0] == -INFINITY ? 0.f : __expf(sv[rt][r][0] - mrow[rt][r]);
        const float p1 = sv[rt][r][1] == -INFINITY ? 0.f : __expf(sv[rt][r][1] - mrow[rt][r]);
        pb[ri * PBS + c16] = (_Float16)p0;
        pb[ri * PBS + 16 + c16] = (_Float16)p1;
        lrow[rt][r] += p0 + p1;  // per-lane partial; rows reduced once after the last key block
      }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    // O += P·V
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
      const h8 pa = *reinterpret_cast<const h8 *>(&sP[wave][rt][c16 * PBS + g * 8]);
#pragma unroll
      for (int t = 0; t < 8; t++) o[rt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, vf[t], o[rt][t], 0, 0, 0);
    }
  }

  _Float16 *O = reinterpret_cast<_Float16 *>(a.out) + (size_t)off * a.ldo + h * HD;
  _Float16 *Olo = a.out_lo ? reinterpret_cast<_Float16 *>(a.out_lo) + (size_t)off * a.ldo + h * HD : nullptr;
  float lsum[RT][4];  // row sums, reduced with every lane active
#pragma unroll
  for (int rt = 0; rt < RT; rt++)
#pragma unroll
    for (int r = 0; r < 4; r++) lsum[rt][r] = row16_sum(lrow[rt][r]);
#pragma unroll
  for (int rt = 0; rt < RT; rt++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int i = iw + rt * 16 + g * 4 + r;
      if (i >= T) continue;
      const float inv = 1.f / lsum[rt][r];
#pragma unroll
      for (int t = 0; t < 8; t++) {
        const float v = o[rt][t][r] * inv;
        const _Float16 hi = (_Float16)v;
        O[(size_t)i * a.ldo + t * 16 + c16] = hi;
        if (Olo) Olo[(size_t)i * a.ldo + t * 16 + c16] = (_Float16)(v - (float)hi);
      }
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
  // FA_ATTN=1: 128-query workgroups (4 waves x 2 row tiles); default: 96-query
  // workgroups (6 waves x 1 row tile, 1.5 waves per SIMD, and a 188-frame
  // window splits 96 + 92 instead of 128 + 60)
  const char *ev = getenv("FA_ATTN");
  if (ev && ev[0] == '1')
    FA_LAUNCH(ps, (relpos_attn_lds_kernel<2, 4>), dim3(cdiv(Tmax, 128), a.H, W), dim3(256), 0, ctx->stream, a, (const _Float16 *)vt, Tp);
  else
    FA_LAUNCH(ps, (relpos_attn_lds_kernel<1, 6>), dim3(cdiv(Tmax, 96), a.H, W), dim3(384), 0, ctx->stream, a, (const _Float16 *)vt, Tp);
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
