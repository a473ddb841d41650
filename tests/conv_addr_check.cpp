// CPU check of the convolution kernels' load addressing (TEST INFRASTRUCTURE).
//
// For every shape given on stdin (B Cin H W Cout KH KW sh sw ph pw dh dw per
// line), every mode, BK in {32, 36}, both operand layouts where allowed and
// several K splits, walks every slot of every chunk of every tile (five
// sampled tiles where an operand has more than six) exactly as
// conv_lds_kernel does (wxx_amd/csrc/conv_addr.h) and checks:
//   * a slot that loads from memory reads inside its tensor;
//   * it reads the element conv_elem() names for its (row, k), and loads zero
//     exactly where conv_elem() says the operand is zero or (row, k) lies
//     outside the tile / the split's K range;
//   * every (row, k) of the tile is written by exactly one slot.
// Prints "ok <checks>" or the first mismatch, exit status 1 on failure.
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "../wxx_amd/csrc/conv_addr.h"

using namespace wxx_conv;

static long long g_checks = 0;

static void fail(const char* what, int mode, bool isp, bool xk, const ConvArgs& a, int x, int k) {
  fprintf(stderr,
          "FAIL %s: mode %d %s %s shape B%d Cin%d H%d W%d Cout%d K%dx%d s%d,%d p%d,%d d%d,%d "
          "kcase %d x %d k %d\n",
          what, mode, isp ? "P" : "Q", xk ? "XK" : "KX", a.B, a.Cin, a.H, a.W, a.Cout, a.KH, a.KW,
          a.sh, a.sw, a.ph, a.pw, a.dh, a.dw, a.kcase, x, k);
  exit(1);
}

static void digits(int mode, const ConvArgs& a, int k, int& t0, int& t1, int& t2) {
  const int R1 = conv_r1(mode, a), R2 = conv_r2(mode, a);
  t0 = k / (R1 * R2);
  t1 = (k - t0 * R1 * R2) / R2;
  t2 = k - (t0 * R1 + t1) * R2;
}

// Expected source of (row x, k) of a tile: -1 for zero, else element offset.
template <int MODE, bool IS_P>
static long long expect(const ConvArgs& a, int x, int k, int kend) {
  if (x >= conv_extent<IS_P>(a) || k >= kend) return -1;
  int t0, t1, t2;
  digits(MODE, a, k, t0, t1, t2);
  long long off;
  if (!conv_elem<MODE, IS_P>(a, x, t0, t1, t2, off)) return -1;
  return off;
}

template <int MODE, bool IS_P, int BK>
static void check_operand(const ConvArgs& a, bool xk) {
  const long long numel = conv_numel<MODE, IS_P>(a);
  const int extent = conv_extent<IS_P>(a);
  const int tiles = (extent + kTile - 1) / kTile;
  const int R1 = conv_r1(MODE, a), R2 = conv_r2(MODE, a), R12 = R1 * R2;
  std::vector<int> hits(kTile * BK);
  for (int splits : {1, 2, 3, 7}) {
    int kps = (a.K + splits - 1) / splits;
    kps = (kps + BK - 1) / BK * BK;
    const int nsplit = (a.K + kps - 1) / kps;
    // every tile of small operands; the first two, a middle and the last two
    // of large ones (their slots differ only by the tile's first row)
    std::vector<int> tlist;
    for (int t = 0; t < tiles; ++t)
      if (tiles <= 6 || t < 2 || t == tiles / 2 || t >= tiles - 2) tlist.push_back(t);
    for (int t : tlist) {
      const int x0 = t * kTile;
      std::vector<XkSlot> slots;
      if (xk)
        for (int w = 0; w < Xk<BK>::kWords; ++w) slots.push_back(xk_slot<MODE, IS_P, BK>(a, x0, w));
      for (int z = 0; z < nsplit; ++z) {
        const int kbeg = z * kps, kend = std::min(a.K, kbeg + kps);
        const int nk = (kend - kbeg + BK - 1) / BK;
        XkUniform u = xk_uniform(MODE, a, kbeg);
        for (int c = 0; c < nk; ++c) {
          const int kbase = kbeg + c * BK, rem = kend - kbase;
          std::fill(hits.begin(), hits.end(), 0);
          if (xk) {
            for (int w = 0; w < Xk<BK>::kWords; ++w) {
              const int xl = w / (BK + 1), col = w - xl * (BK + 1);
              int off = 0;
              const bool ld = xk_src<MODE, IS_P>(a, slots[w], u, kbase, rem, off);
              if (xl >= kTile || col >= BK) {
                if (ld) fail("padding slot loads", MODE, IS_P, xk, a, x0 + xl, kbase + col);
                continue;
              }
              ++hits[xl * BK + col];
              const long long e = expect<MODE, IS_P>(a, x0 + xl, kbase + col, kend);
              if (ld && (off < 0 || off >= numel))
                fail("out of bounds", MODE, IS_P, xk, a, x0 + xl, kbase + col);
              if ((ld ? off : -1LL) != e) fail("wrong element", MODE, IS_P, xk, a, x0 + xl, kbase + col);
              ++g_checks;
            }
            xk_advance(MODE, a, u, BK);
          } else if (a.kcase != 0 || (MODE == kFwd && IS_P)) {
            // KX rows as slots (row = chunk column), as the kernels build them
            for (int r = 0; r < BK; ++r) {
              for (int l = 0; l < kTile; ++l) {
                const XkSlot sl = kx_slot<MODE, IS_P, BK>(a, x0, l, r);
                int off = 0;
                const bool ld = xk_src<MODE, IS_P>(a, sl, u, kbase, rem, off);
                ++hits[l * BK + r];
                const long long e = expect<MODE, IS_P>(a, x0 + l, kbase + r, kend);
                if (ld && (off < 0 || off >= numel)) fail("out of bounds", MODE, IS_P, xk, a, x0 + l, kbase + r);
                if ((ld ? off : -1LL) != e) fail("wrong element", MODE, IS_P, xk, a, x0 + l, kbase + r);
                ++g_checks;
              }
            }
            xk_advance(MODE, a, u, BK);
          } else {
            for (int r = 0; r < BK; ++r) {
              const int k = kbase + r;
              int t0, t1, t2;
              digits(MODE, a, k, t0, t1, t2);
              for (int l = 0; l < kTile; ++l) {
                const KxCol cd = kx_col<MODE, IS_P>(a, x0 + l);
                long long off = 0;
                const bool ld = k < kend && kx_src<MODE, IS_P>(a, cd, k, t0, t1, t2, off);
                ++hits[l * BK + r];
                const long long e = expect<MODE, IS_P>(a, x0 + l, k, kend);
                if (ld && (off < 0 || off >= numel)) fail("out of bounds", MODE, IS_P, xk, a, x0 + l, k);
                if ((ld ? off : -1LL) != e) fail("wrong element", MODE, IS_P, xk, a, x0 + l, k);
                ++g_checks;
              }
            }
          }
          for (int h : hits)
            if (h != 1) fail("tile word not written exactly once", MODE, IS_P, xk, a, x0, kbase);
        }
      }
    }
  }
  (void)R12;
}

template <int MODE, int BK>
static void check_mode(ConvArgs a) {
  const int R2 = conv_r2(MODE, a), R12 = conv_r1(MODE, a) * R2;
  a.kcase = BK % R12 == 0 ? 1 : (MODE == kDw && R12 % BK == 0 && BK % R2 == 0) ? 2 : 0;
  conv_prepare(MODE, a);
  check_operand<MODE, true, BK>(a, false);
  check_operand<MODE, false, BK>(a, false);
  if (MODE == kFwd || a.kcase) check_operand<MODE, true, BK>(a, true);
  if (a.kcase) check_operand<MODE, false, BK>(a, true);
}

// FastDiv against the division operator: every divisor up to 4096 with
// dividends near multiples of it, and large divisors with extreme dividends.
static void check_fastdiv() {
  unsigned long long st = 12345;
  auto rnd = [&]() { st = st * 6364136223846793005ULL + 1442695040888963407ULL; return (int)(st >> 33); };
  for (int d = 1; d <= 4096; ++d) {
    const FastDiv f = make_fastdiv(d);
    for (int m = 0; m < 64; ++m) {
      const long long base = (long long)d * (rnd() % ((0x7fffffff / d) + 1));
      for (int e = -1; e <= 1; ++e) {
        const long long x = base + e;
        if (x < 0 || x > 0x7fffffff) continue;
        if (fdiv((int)x, f) != (int)(x / d)) { fprintf(stderr, "FAIL fdiv %lld / %d\n", x, d); exit(1); }
      }
    }
  }
  for (int n = 0; n < 200000; ++n) {
    const int d = 1 + rnd() % 0x7ffffffe;
    const FastDiv f = make_fastdiv(d);
    for (int x : {0, 1, d - 1, d, 0x7fffffff, rnd()})
      if (x >= 0 && fdiv(x, f) != x / d) { fprintf(stderr, "FAIL fdiv %d / %d\n", x, d); exit(1); }
  }
}

int main() {
  check_fastdiv();
  int B, Cin, H, W, Cout, KH, KW, sh, sw, ph, pw, dh, dw;
  int shapes = 0;
  while (scanf("%d %d %d %d %d %d %d %d %d %d %d %d %d", &B, &Cin, &H, &W, &Cout, &KH, &KW, &sh,
               &sw, &ph, &pw, &dh, &dw) == 13) {
    ConvArgs a{};
    a.B = B; a.Cin = Cin; a.H = H; a.W = W; a.Cout = Cout; a.KH = KH; a.KW = KW;
    a.sh = sh; a.sw = sw; a.ph = ph; a.pw = pw; a.dh = dh; a.dw = dw;
    a.Ho = (H + 2 * ph - dh * (KH - 1) - 1) / sh + 1;
    a.Wo = (W + 2 * pw - dw * (KW - 1) - 1) / sw + 1;
    ConvArgs f = a;  // forward
    f.I = Cout; f.J = B * a.Ho * a.Wo; f.K = Cin * KH * KW;
    ConvArgs x = a;  // dX
    x.I = Cin; x.J = B * H * W; x.K = Cout * KH * KW;
    ConvArgs w = a;  // dW
    w.I = Cout; w.J = Cin * KH * KW; w.K = B * a.Ho * a.Wo;
    check_mode<kFwd, 32>(f);
    check_mode<kFwd, 36>(f);
    check_mode<kDx, 32>(x);
    check_mode<kDx, 36>(x);
    check_mode<kDw, 32>(w);
    ++shapes;
  }
  printf("ok %d shapes %lld checks\n", shapes, g_checks);
  return 0;
}
