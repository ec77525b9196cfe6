"""The decoder's joint kernel with two windows per wave (16 window slots per
workgroup): a variant of fluidaudio-web_amd/csrc/tdt.hip's tdt_joint_kernel that
was run on the GPU once, made an illegal memory access on its first decode of
more than 16 windows, and was removed.  `variant_source()` returns tdt.hip with
this kernel in place of the shipped one (and its launch at 8 waves per
workgroup), for the CPU execution of kernel sources (tests/emu), which runs it
under AddressSanitizer.  Test infrastructure: nothing here is built into the
library."""
from __future__ import annotations

import os

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
TDT = os.path.join(ROOT, "fluidaudio-web_amd", "csrc", "tdt.hip")

KERNEL = r'''constexpr int RS_KC = 64, RS_S = 4, RS_WAVES = 8, RS_WPW = 2;  // rows per chunk, chunks in flight, waves per block, windows per wave
constexpr int RS_SLOTS = RS_WAVES * RS_WPW;                     // windows per block

// Wave = two selected windows, lane = one column of a 64-column slab: every
// lane runs two independent in-order chains over the 640 hidden units (one per
// window) on the same weights, so each weight read from LDS feeds two chains
// and the two chains' dependent adds interleave.  The windows' input vectors
// are wave-uniform and read with scalar loads (SGPR operands of the
// multiplies; measured 18.7 us per step against 29.0 with the vector staged in
// LDS and read as broadcasts); the slab's rows are streamed global->LDS by
// global_load_lds_dwordx4 in chunks of 64 rows, RS_S chunks in flight, and
// shared by the block's 16 windows.  W rows must be 16-byte aligned and the
// slab must lie inside every row.
// Selected = windows with frames left; per-slab token maximum, and the
// duration maximum in the last slab.
__global__ __launch_bounds__(64 * RS_WAVES) void tdt_joint_kernel(const float *__restrict__ W, int ldw, int ncols, const float *__restrict__ bias,
                                                                  const float *__restrict__ xsrc, TdtState st, int n) {
  __shared__ __attribute__((aligned(1024))) float ws[RS_S][RS_KC][TJB];
  __shared__ int lst[RS_SLOTS], lcnt;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int slab = blockIdx.x, col = slab * TJB + lane;
  if (wave == 0) {
    const bool sel = lane < n && st.win[lane].t < st.win[lane].T;
    const unsigned long long m = __ballot(sel);
    const int first = blockIdx.y * RS_SLOTS, rank = __popcll(m & ((1ull << lane) - 1ull));
    if (sel && rank >= first && rank < first + RS_SLOTS) lst[rank - first] = lane;
    if (lane == 0) lcnt = min(max(__popcll(m) - first, 0), RS_SLOTS);
  }
  __syncthreads();
  const int cnt = lcnt;
  if (cnt == 0) return;  // uniform
  const uint32_t sb = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) char *)&ws[0][0][0]);
  // a chunk is 64 rows x 256 B = 16 copies of 1 KB (4 rows each), two per wave
  const float *wsrc = W + (size_t)(lane >> 4) * ldw + slab * TJB + (lane & 15) * 4;
  auto issue = [&](int ch) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int ins = wave * 2 + i;
      tdt_dma16(wsrc + (size_t)(ch * RS_KC + ins * 4) * ldw, sb + (ch % RS_S) * (RS_KC * TJB * 4) + ins * 1024);
    }
  };
  constexpr int NCH = TH / RS_KC;
#pragma unroll
  for (int ch = 0; ch < RS_S - 1; ch++) issue(ch);
  // this wave's windows: slots 2 wave and 2 wave + 1 (a missing second one
  // repeats the first, its result unused)
  const bool work = RS_WPW * wave < cnt, two = RS_WPW * wave + 1 < cnt;
  const int w0 = __builtin_amdgcn_readfirstlane(lst[work ? RS_WPW * wave : 0]);
  const int w1 = __builtin_amdgcn_readfirstlane(lst[two ? RS_WPW * wave + 1 : (work ? RS_WPW * wave : 0)]);
  const float *xw0 = xsrc + (size_t)w0 * TH, *xw1 = xsrc + (size_t)w1 * TH;  // wave-uniform: scalar loads, SGPR operands
  const bool valid = col < ncols;
  float acc0 = valid ? bias[col] : 0.f, acc1 = acc0;
  for (int ch = 0; ch < NCH; ch++) {
    const int newer = min(RS_S - 2, NCH - 1 - ch);  // copies issued after chunk ch, per wave: 2 each
    if (newer >= 2) tdt_wait_vmcnt<4>();
    else if (newer == 1) tdt_wait_vmcnt<2>();
    else tdt_wait_vmcnt<0>();
    __syncthreads();  // chunk ch visible to every wave; the stage of chunk ch - 1 is free
    if (ch + RS_S - 1 < NCH) issue(ch + RS_S - 1);
    if (work) {
      const float *wr = &ws[ch % RS_S][0][lane];
      const int k0 = ch * RS_KC;
      float wA[16], wB[16], xA0[16], xB0[16], xA1[16], xB1[16];
      auto ld = [&](int kk, float(&wv)[16], float(&xv0)[16], float(&xv1)[16]) {
#pragma unroll
        for (int u = 0; u < 16; u++) wv[u] = wr[(kk + u) * TJB];
#pragma unroll
        for (int u = 0; u < 16; u++) xv0[u] = xw0[k0 + kk + u];
#pragma unroll
        for (int u = 0; u < 16; u++) xv1[u] = xw1[k0 + kk + u];
      };
      auto sum = [&](const float(&wv)[16], const float(&xv0)[16], const float(&xv1)[16]) {
#pragma unroll
        for (int u = 0; u < 16; u++) {
          acc0 = acc0 + xv0[u] * wv[u];
          acc1 = acc1 + xv1[u] * wv[u];
        }
      };
      ld(0, wA, xA0, xA1);
      ld(16, wB, xB0, xB1);
      sum(wA, xA0, xA1);
      ld(32, wA, xA0, xA1);
      sum(wB, xB0, xB1);
      ld(48, wB, xB0, xB1);
      sum(wA, xA0, xA1);
      sum(wB, xB0, xB1);
    }
  }
  if (!work) return;
  auto finish = [&](float acc, int w) {
    float bv = (valid && col < TV) ? acc : -INFINITY;
    int bi = (valid && col < TV) ? col : 0x7fffffff;
#pragma unroll
    for (int sh = 32; sh > 0; sh >>= 1) {
      const float ov = __shfl_xor(bv, sh);
      const int oi = __shfl_xor(bi, sh);
      if (better(ov, oi, bv, bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if (lane == 0) {
      st.pv[w * TNB + slab] = bv;
      st.pi[w * TNB + slab] = bi;
    }
    if (slab == TNB - 1) {
      float dv = (valid && col >= TV) ? acc : -INFINITY;
      int di = (valid && col >= TV) ? col - TV : 0x7fffffff;
#pragma unroll
      for (int sh = 32; sh > 0; sh >>= 1) {
        const float ov = __shfl_xor(dv, sh);
        const int oi = __shfl_xor(di, sh);
        if (better(ov, oi, dv, di)) {
          dv = ov;
          di = oi;
        }
      }
      if (lane == 0) {
        st.dv[w] = dv;
        st.di[w] = di;
      }
    }
  };
  finish(acc0, w0);
  if (two) finish(acc1, w1);
}

'''


def variant_source() -> str:
    s = open(TDT).read()
    a = s.index("constexpr int RS_KC = 64, RS_S = 4, RS_SLOTS = 8;")
    b = s.index("// Pred projection of the windows that emitted")
    s = s[:a] + KERNEL + s[b:]
    old = "FA_LAUNCH(ps, tdt_joint_kernel, dim3(TNB, cdiv(n, RS_SLOTS)), dim3(64 * RS_SLOTS), 0,"
    assert old in s, "the shipped joint launch changed"
    return s.replace(old, "FA_LAUNCH(ps, tdt_joint_kernel, dim3(TNB, cdiv(n, RS_SLOTS)), dim3(64 * RS_WAVES), 0,")
