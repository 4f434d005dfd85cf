// gemvk.hip -- host launchers of the few-row VALU GEMV (gemvk.h), in a
// translation unit of their own so the kernel instantiations compile in
// parallel with the rest of the library.
#include "gemvk.h"

namespace wc {

// Few-row VALU GEMV (k_gemvk): 2..8 input rows, every K a multiple of 512,
// every segment normed or none.  S (512-wide steps per wave) is the smallest
// that keeps the block at most kGkWaveCap waves with every wave inside one
// segment (one segment: the last wave may run past its end).
constexpr int kGkWaveCap = 12;
template <int R, bool PAIR, int NIN, int S, int MM, int XB, int GB>
static bool launch_gemvk_w(const GemvArgs& a, int waves, hipStream_t s) {
  const dim3 grid((a.N + R - 1) / R), block(waves * kWave);
  if (waves <= 4) {
    hipLaunchKernelGGL((k_gemvk<R, PAIR, NIN, S, MM, XB, GB, 4>), grid, block, 0, s, a);
  } else if (waves <= 8) {
    hipLaunchKernelGGL((k_gemvk<R, PAIR, NIN, S, MM, XB, GB, 8>), grid, block, 0, s, a);
  } else {
    // twelve waves cap the registers at 168: no room for two steps of eight rows
    if constexpr (S * MM > 8) return false;
    else hipLaunchKernelGGL((k_gemvk<R, PAIR, NIN, S, MM, XB, GB, 12>), grid, block, 0, s, a);
  }
  return true;
}
template <int R, bool PAIR, int NIN, int S, int XB, int GB>
static bool launch_gemvk_m(const GemvArgs& a, int waves, hipStream_t s) {
  if (a.M <= 4) return launch_gemvk_w<R, PAIR, NIN, S, 4, XB, GB>(a, waves, s);
  if (a.M <= 6) return launch_gemvk_w<R, PAIR, NIN, S, 6, XB, GB>(a, waves, s);
  return launch_gemvk_w<R, PAIR, NIN, S, 8, XB, GB>(a, waves, s);
}
// R: output rows per block, the wide choice (twice the rows) on one step per wave only
template <bool PAIR, int NIN, int XB, int GB>
static bool launch_gemvk_g(const GemvArgs& a, int S, int waves, bool wide, hipStream_t s) {
  constexpr int RS = PAIR ? 2 : 4;
  if (S == 1) {
    if (wide) return launch_gemvk_m<2 * RS, PAIR, NIN, 1, XB, GB>(a, waves, s);
    return launch_gemvk_m<RS, PAIR, NIN, 1, XB, GB>(a, waves, s);
  }
  if (S == 2) return launch_gemvk_m<RS, PAIR, NIN, 2, XB, GB>(a, waves, s);
  return false;
}
// Measured at the Qwen3-1.7B drafter shape with 5 host rows, 3 live
// (fuse, QKV, o, down: 9.0 / 12.4 / 5.0 / 8.6 us against 14.1 / 14.6 / 7.5 /
// 13.1 on the MFMA kernels).  The gate / up pair stays on the MFMA kernel
// (14.3 us here against 14.2 there).  Blocks of twelve waves take twice the
// rows (fuse, down: fewer blocks for the same bytes in flight).
template <int NIN, int XB>
static bool launch_gemvk(const GemvArgs& a, hipStream_t s) {
  if (a.M < 2 || a.M > 8 || a.xn_out || a.epi == kEpiArgmax || a.n_in != NIN) return false;
  if (a.fin_gain && (!a.fin_counter || !a.fin_out)) return false;
  int gb = 0, st[kMaxIn] = {0, 0, 0};
  for (int i = 0; i < NIN; ++i) {
    if (a.in[i].K % 512 != 0 || a.in[i].K == 0) return false;
    st[i] = a.in[i].K / 512;
    if (a.in[i].gain) gb |= 1 << i;
  }
  constexpr int kAll = (1 << NIN) - 1;
  if (gb != 0 && gb != kAll) return false;
  int S = 0, waves = 0;
  for (int c : {1, 2}) {
    bool ok = true;
    int wv = 0;
    for (int i = 0; i < NIN; ++i) {
      if (NIN > 1 && st[i] % c != 0) ok = false;
      wv += (st[i] + c - 1) / c;
    }
    if (ok && wv <= kGkWaveCap) {
      S = c;
      waves = wv;
      break;
    }
  }
  if (S == 0) return false;
  const bool wide = waves >= 12;
  if (gb) return launch_gemvk_g<false, NIN, XB, kAll>(a, S, waves, wide, s);
  // gain-free inputs: o_proj / down, and the fuse without feature norms
  if constexpr (NIN == 2) return false;
  else return launch_gemvk_g<false, NIN, XB, 0>(a, S, waves, wide, s);
}

bool launch_gemvk_any(const GemvArgs& a, bool pair, int xb, hipStream_t s) {
  if (pair) return false;
  if (a.n_in == 1 && xb == 0) return launch_gemvk<1, 0>(a, s);
  if (a.n_in == 2 && xb == 2) return launch_gemvk<2, 2>(a, s);
  if (a.n_in == 3 && xb == 0) return launch_gemvk<3, 0>(a, s);
  if (a.n_in == 3 && xb == 7) return launch_gemvk<3, 7>(a, s);
  return false;
}

}  // namespace wc
