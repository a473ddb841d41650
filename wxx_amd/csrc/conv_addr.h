// Operand addressing of the implicit-GEMM convolution kernels (conv.hip).
//
// Plain C++ shared by the gfx950 kernels, the host-side layout choice and a
// CPU checker (tests/test_conv_addr.py) that compares every load source the
// kernels would compute against conv_elem() and the tensor bounds.  Define
// WXX_HD before including to add __host__ __device__.
//
// Each convolution mode is one GEMM  Out[i][j] = sum_k P[i][k] Q[k][j]:
//   forward: i = co, j = (b, oh, ow), k = (ci, kh, kw); P = W, Q = im2col(X)
//   dX:      i = ci, j = (b, ih, iw), k = (co, kh, kw); P = W^T per tap, Q = gather(dY)
//   dW:      i = co, j = (ci, kh, kw), k = (b, oh, ow); P = dY, Q = im2col(X)^T
// k is written as digits (t0, t1, t2) in radices (R1, R2):
//   k = (t0 R1 + t1) R2 + t2,  (R1, R2) = (KH, KW) for forward / dX, (Ho, Wo) for dW.
//
// An operand tile (64 rows x of i or j, BK columns of k per chunk) is
// written to LDS by wave-wide loads: the n-th load of a wave fills 64
// consecutive LDS words, one per lane, from any 64 addresses.  Two layouts:
//   KX  k-major [BK][64 + 2]: an instruction is one row k, lanes run along x.
//       The row's digits are wave-uniform; each lane keeps its column's data
//       (in cases 1 and 2 below a row is a slot like an XK word).
//   XK  x-major [64][BK + 1]: lanes run along k (odd row stride, so the MFMA
//       operand reads, 32 lanes down a column, hit 32 different banks).  Each
//       lane's slot (x, c) is fixed for the whole K loop; per chunk only a
//       wave-uniform offset is added.  That needs every slot's digits to be
//       a fixed part plus a uniform part:
//         case 1  BK % R12 == 0: chunks start at t1 = t2 = 0, so (t1, t2) are
//                 fixed per slot and t0 = t0_u + t0_s;
//         case 2  R12 % BK == 0 and BK % R2 == 0 (dW only): t0 = t0_u is
//                 uniform, t1 = t1_u + t1_s, t2 fixed; the row bound of the
//                 X gather is then checked per chunk.
//       The forward's P (W, contiguous along k) needs no digits at all.
// Whichever layout touches fewer 128-byte lines per instruction for the
// launch's shape is chosen on the host (conv_lines()).
#pragma once

#ifndef WXX_HD
#define WXX_HD inline
#endif

namespace wxx_conv {

enum { kFwd = 0, kDx = 1, kDw = 2 };
constexpr int kTile = 64;  // rows of an operand tile (BI = BJ = 64)

// Division by a runtime divisor d >= 1 as a multiply and shift (Granlund and
// Montgomery, "Division by invariant integers using multiplication", 1994):
// with l = ceil(log2 d) and m = floor(2^(31 + l) / d) + 1, floor(x / d) =
// (x m) >> (31 + l) for 0 <= x < 2^31.
struct FastDiv {
  unsigned long long m;
  int s;
};

inline FastDiv make_fastdiv(int d) {
  int l = 0;
  while ((1LL << l) < d) ++l;
  FastDiv f;
  f.s = 31 + l;
  f.m = ((1ULL << f.s) / (unsigned long long)d) + 1;
  return f;
}

WXX_HD int fdiv(int x, const FastDiv& f) {
  return (int)(((unsigned long long)(unsigned)x * f.m) >> f.s);
}

struct ConvArgs {
  const float* P;
  const float* Q;
  const float* bias;
  float* out;  // final tensor (splits == 1) or partials [splits][I][J]
  int B, Cin, H, W, Cout, KH, KW, Ho, Wo, sh, sw, ph, pw, dh, dw;
  int I, J, K;
  int kps;  // K elements per split (multiple of BK)
  int splits;
  int tiles_i, tiles_j;
  int kcase;  // XK decomposition (1 or 2, see above); 0 where only the forward's P may be XK
  const float* zero;  // a device word of zeros: the source of every zero element
  // divisors of the index arithmetic (conv_prepare)
  FastDiv dR12, dR2, dHoWo, dWo, dHW, dW, dKK, dKW, dsh, dsw;
};

// Divisors of the index arithmetic (host, once per launch).
inline void conv_prepare(int mode, ConvArgs& a) {
  const int R1 = mode == kDw ? a.Ho : a.KH, R2 = mode == kDw ? a.Wo : a.KW;
  a.dR12 = make_fastdiv(R1 * R2);
  a.dR2 = make_fastdiv(R2);
  a.dHoWo = make_fastdiv(a.Ho * a.Wo);
  a.dWo = make_fastdiv(a.Wo);
  a.dHW = make_fastdiv(a.H * a.W);
  a.dW = make_fastdiv(a.W);
  a.dKK = make_fastdiv(a.KH * a.KW);
  a.dKW = make_fastdiv(a.KW);
  a.dsh = make_fastdiv(a.sh);
  a.dsw = make_fastdiv(a.sw);
}

WXX_HD int conv_r1(int mode, const ConvArgs& a) { return mode == kDw ? a.Ho : a.KH; }
WXX_HD int conv_r2(int mode, const ConvArgs& a) { return mode == kDw ? a.Wo : a.KW; }

// Rows of the operand (i extent for P, j extent for Q).
template <bool IS_P>
WXX_HD int conv_extent(const ConvArgs& a) {
  return IS_P ? a.I : a.J;
}

// The definition: element offset of P[x][k] (IS_P) or Q[k][x] inside its
// tensor for k = digits (t0, t1, t2); false where the operand is zero
// (padding, stride gaps).  Validity never depends on t0, and the offset is
// affine in t0 (coefficient conv_a0) and, for dW, in t1 (conv_a1).
template <int MODE, bool IS_P>
WXX_HD bool conv_elem(const ConvArgs& a, int x, int t0, int t1, int t2, long long& off) {
  const int HW = a.H * a.W, HoWo = a.Ho * a.Wo, KK = a.KH * a.KW;
  if (MODE == kFwd) {
    if (IS_P) {
      off = (long long)x * a.K + ((long long)t0 * a.KH + t1) * a.KW + t2;
      return true;
    }
    const int b = x / HoWo, pos = x - b * HoWo, oh = pos / a.Wo, ow = pos - oh * a.Wo;
    const int iy = oh * a.sh - a.ph + t1 * a.dh, ix = ow * a.sw - a.pw + t2 * a.dw;
    if ((unsigned)iy >= (unsigned)a.H || (unsigned)ix >= (unsigned)a.W) return false;
    off = ((long long)b * a.Cin + t0) * HW + (long long)iy * a.W + ix;
    return true;
  }
  if (MODE == kDx) {
    if (IS_P) {
      off = ((long long)t0 * a.Cin + x) * KK + t1 * a.KW + t2;
      return true;
    }
    const int b = x / HW, pos = x - b * HW, ih = pos / a.W, iw = pos - ih * a.W;
    const int th = ih + a.ph - t1 * a.dh, tw = iw + a.pw - t2 * a.dw;
    if (th < 0 || tw < 0) return false;
    const int oh = th / a.sh, ow = tw / a.sw;
    if (oh * a.sh != th || ow * a.sw != tw || oh >= a.Ho || ow >= a.Wo) return false;
    off = ((long long)b * a.Cout + t0) * HoWo + (long long)oh * a.Wo + ow;
    return true;
  }
  if (IS_P) {
    off = ((long long)t0 * a.Cout + x) * HoWo + (long long)t1 * a.Wo + t2;
    return true;
  }
  const int ci = x / KK, kk = x - ci * KK, kh = kk / a.KW, kw = kk - kh * a.KW;
  const int iy = t1 * a.sh - a.ph + kh * a.dh, ix = t2 * a.sw - a.pw + kw * a.dw;
  if ((unsigned)iy >= (unsigned)a.H || (unsigned)ix >= (unsigned)a.W) return false;
  off = ((long long)t0 * a.Cin + ci) * HW + (long long)iy * a.W + ix;
  return true;
}

template <int MODE, bool IS_P>
WXX_HD int conv_a0(const ConvArgs& a) {
  if (MODE == kFwd) return IS_P ? a.KH * a.KW : a.H * a.W;
  if (MODE == kDx) return IS_P ? a.Cin * a.KH * a.KW : a.Ho * a.Wo;
  return IS_P ? a.Cout * a.Ho * a.Wo : a.Cin * a.H * a.W;
}
template <int MODE, bool IS_P>
WXX_HD int conv_a1(const ConvArgs& a) {
  return MODE == kDw ? (IS_P ? a.Wo : a.sh * a.W) : 0;
}

// Elements of the operand's tensor (for bounds checks).
template <int MODE, bool IS_P>
WXX_HD long long conv_numel(const ConvArgs& a) {
  const long long x = (long long)a.B * a.Cin * a.H * a.W;
  const long long y = (long long)a.B * a.Cout * a.Ho * a.Wo;
  const long long w = (long long)a.Cout * a.Cin * a.KH * a.KW;
  if (MODE == kFwd) return IS_P ? w : x;
  if (MODE == kDx) return IS_P ? w : y;
  return IS_P ? y : x;
}

// ---- XK slots -------------------------------------------------------------
// Wave loads per operand tile in the XK layout, padded to a multiple
// of the 4 waves; and per wave.
template <int BK>
struct Xk {
  static constexpr int kRow = BK + 1;
  static constexpr int kInst = ((kTile * kRow + 63) / 64 + 3) / 4 * 4;
  static constexpr int kPerWave = kInst / 4;
  static constexpr int kWords = kInst * 64;
};

constexpr int kDeadSlot = 1 << 29;  // c of a slot that always loads zero

struct XkSlot {
  int off;  // element offset of the fixed part (meaningful when c < kDeadSlot)
  int c;    // column within the chunk; kDeadSlot when the slot always loads zero
  int iy;   // case 2, dW's Q: fixed part of the X row, checked per chunk
};

// A slot's fixed part is the sum of an entry of its row x (SlotX) and an
// entry of its chunk column c (SlotC): the kernels compute the 64 row and BK
// column entries of a tile once, then each slot from one entry of each.
struct SlotX {
  int base, y, x, ok;
};
struct SlotC {
  int base, y, x, ok;
};

template <int MODE, bool IS_P>
WXX_HD SlotX slot_x(const ConvArgs& a, int x) {
  SlotX e;
  e.ok = x < conv_extent<IS_P>(a);
  const int xx = e.ok ? x : 0;
  const int HW = a.H * a.W, HoWo = a.Ho * a.Wo, KK = a.KH * a.KW;
  e.y = e.x = 0;
  if (IS_P) {
    e.base = xx * (MODE == kFwd ? a.K : (MODE == kDx ? KK : HoWo));
  } else if (MODE == kFwd) {
    const int b = fdiv(xx, a.dHoWo), pos = xx - b * HoWo, oh = fdiv(pos, a.dWo);
    e.base = b * a.Cin * HW;
    e.y = oh * a.sh - a.ph;
    e.x = (pos - oh * a.Wo) * a.sw - a.pw;
  } else if (MODE == kDx) {
    const int b = fdiv(xx, a.dHW), pos = xx - b * HW, ih = fdiv(pos, a.dW);
    e.base = b * a.Cout * HoWo;
    e.y = ih + a.ph;
    e.x = pos - ih * a.W + a.pw;
  } else {
    const int ci = fdiv(xx, a.dKK), kk = xx - ci * KK, kh = fdiv(kk, a.dKW);
    e.base = ci * HW;
    e.y = kh * a.dh - a.ph;
    e.x = (kk - kh * a.KW) * a.dw - a.pw;
  }
  return e;
}

// Column c of a chunk: its digits are (t0s, t1s, t2s) of c in case 1 and
// (0, c / R2, c % R2) in case 2 (the forward's P takes c itself).
template <int MODE, bool IS_P>
WXX_HD SlotC slot_c(const ConvArgs& a, int c, int BK) {
  SlotC e;
  e.ok = c < BK;
  e.base = e.y = e.x = 0;
  if (!e.ok) return e;
  if (MODE == kFwd && IS_P) {
    e.base = c;
    return e;
  }
  const int R2 = conv_r2(MODE, a), R12 = conv_r1(MODE, a) * R2;
  int t0s, t1s, t2s;
  if (a.kcase == 1) {
    t0s = fdiv(c, a.dR12);
    const int r = c - t0s * R12;
    t1s = fdiv(r, a.dR2);
    t2s = r - t1s * R2;
  } else {
    t0s = 0;
    t1s = fdiv(c, a.dR2);
    t2s = c - t1s * R2;
  }
  const int HW = a.H * a.W, HoWo = a.Ho * a.Wo, KK = a.KH * a.KW;
  if (MODE == kFwd) {
    e.base = t0s * HW;
    e.y = t1s * a.dh;
    e.x = t2s * a.dw;
  } else if (MODE == kDx) {
    if (IS_P) {
      e.base = t0s * a.Cin * KK + t1s * a.KW + t2s;
    } else {
      e.base = t0s * HoWo;
      e.y = t1s * a.dh;
      e.x = t2s * a.dw;
    }
  } else {
    if (IS_P) {
      e.base = t0s * a.Cout * HoWo + t1s * a.Wo + t2s;
    } else {
      e.base = t0s * a.Cin * HW;
      e.y = t1s * a.sh;
      e.x = t2s * a.sw;
    }
  }
  return e;
}

// The slot of row entry X and column entry Cc (column index c).
template <int MODE, bool IS_P>
WXX_HD XkSlot slot_make(const ConvArgs& a, const SlotX& X, const SlotC& Cc, int c) {
  XkSlot s;
  s.off = 0;
  s.iy = 0;
  s.c = kDeadSlot;
  if (!X.ok || !Cc.ok) return s;
  if (IS_P) {
    s.off = X.base + Cc.base;
    s.c = c;
    return s;
  }
  if (MODE == kFwd) {
    const int iy = X.y + Cc.y, ix = X.x + Cc.x;
    if ((unsigned)iy >= (unsigned)a.H || (unsigned)ix >= (unsigned)a.W) return s;
    s.off = X.base + Cc.base + iy * a.W + ix;
  } else if (MODE == kDx) {
    const int th = X.y - Cc.y, tw = X.x - Cc.x;
    if (a.sh == 1 && a.sw == 1) {
      if ((unsigned)th >= (unsigned)a.Ho || (unsigned)tw >= (unsigned)a.Wo) return s;
      s.off = X.base + Cc.base + th * a.Wo + tw;
    } else {
      if (th < 0 || tw < 0) return s;
      const int oh = fdiv(th, a.dsh), ow = fdiv(tw, a.dsw);
      if (oh * a.sh != th || ow * a.sw != tw || oh >= a.Ho || ow >= a.Wo) return s;
      s.off = X.base + Cc.base + oh * a.Wo + ow;
    }
  } else {
    const int iy = X.y + Cc.y, ix = X.x + Cc.x;
    if ((unsigned)ix >= (unsigned)a.W) return s;
    if (a.kcase == 2) {
      s.iy = iy;  // iy + t1_u sh is checked per chunk
    } else if ((unsigned)iy >= (unsigned)a.H) {
      return s;
    }
    s.off = X.base + Cc.base + iy * a.W + ix;
  }
  s.c = c;
  return s;
}

// Slot of word w (= 64 * instruction + lane) of an XK tile whose first row
// is x0.
template <int MODE, bool IS_P, int BK>
WXX_HD XkSlot xk_slot(const ConvArgs& a, int x0, int w) {
  const int xl = w / (BK + 1), c = w - xl * (BK + 1);
  if (xl >= kTile) {
    XkSlot s;
    s.off = s.iy = 0;
    s.c = kDeadSlot;
    return s;
  }
  return slot_make<MODE, IS_P>(a, slot_x<MODE, IS_P>(a, x0 + xl), slot_c<MODE, IS_P>(a, c, BK), c);
}

// Slot of row `row` of a KX tile (lane = column x0 + lane): the same
// decomposition with the row as the chunk column.
template <int MODE, bool IS_P, int BK>
WXX_HD XkSlot kx_slot(const ConvArgs& a, int x0, int lane, int row) {
  return slot_make<MODE, IS_P>(a, slot_x<MODE, IS_P>(a, x0 + lane), slot_c<MODE, IS_P>(a, row, BK),
                               row);
}

// Wave-uniform digit state of the chunk that starts at k = kbase.
struct XkUniform {
  int t0, t1;
};

WXX_HD XkUniform xk_uniform(int mode, const ConvArgs& a, int kbase) {
  const int R2 = conv_r2(mode, a), R12 = conv_r1(mode, a) * R2;
  XkUniform u;
  u.t0 = fdiv(kbase, a.dR12);
  u.t1 = fdiv(kbase - u.t0 * R12, a.dR2);  // 0 in case 1
  return u;
}

// Advance by one chunk of BK.
WXX_HD void xk_advance(int mode, const ConvArgs& a, XkUniform& u, int BK) {
  const int R1 = conv_r1(mode, a), R2 = conv_r2(mode, a), R12 = R1 * R2;
  if (a.kcase == 1) {
    u.t0 += BK / R12;
  } else {
    u.t1 += BK / R2;
    if (u.t1 >= R1) {
      u.t1 -= R1;
      u.t0 += 1;
    }
  }
}

// Wave-uniform part of the offset of every slot of a chunk.
template <int MODE, bool IS_P>
WXX_HD int xk_uoff(const ConvArgs& a, const XkUniform& u, int kbase) {
  if (MODE == kFwd && IS_P) return kbase;
  return conv_a0<MODE, IS_P>(a) * u.t0 + conv_a1<MODE, IS_P>(a) * u.t1;
}

// Does the slot load from memory in this chunk?  lim = the chunk's valid
// columns (kDeadSlot for a full chunk).
template <int MODE, bool IS_P>
WXX_HD bool xk_valid(const ConvArgs& a, const XkSlot& s, const XkUniform& u, int lim) {
  bool ok = s.c < lim;
  if (MODE == kDw && !IS_P) {
    if (a.kcase == 2) ok = ok && (unsigned)(s.iy + u.t1 * a.sh) < (unsigned)a.H;
  }
  return ok;
}

// Source element offset of a slot for the chunk with uniform state u and
// rem = kend - kbase valid columns; false where the slot loads zero.
template <int MODE, bool IS_P>
WXX_HD bool xk_src(const ConvArgs& a, const XkSlot& s, const XkUniform& u, int kbase, int rem,
                   int& off) {
  if (!xk_valid<MODE, IS_P>(a, s, u, rem)) return false;
  off = s.off + xk_uoff<MODE, IS_P>(a, u, kbase);
  return true;
}

// ---- KX columns -----------------------------------------------------------
// Per-lane data of column x, fixed over the K loop.  A row k's source offset
// is lo + kx_uoff(k) (wave-uniform part), loaded where kx_valid() holds.
struct KxCol {
  int ok;    // x inside the operand
  int y, x;  // forward: (oh sh - ph, ow sw - pw); dX: (ih + ph, iw + pw); dW: (kh dh - ph, kw dw - pw)
  int lo;    // lane part of the offset
};

template <int MODE, bool IS_P>
WXX_HD KxCol kx_col(const ConvArgs& a, int x) {
  KxCol cd;
  cd.ok = x < conv_extent<IS_P>(a);
  const int xx = cd.ok ? x : 0;
  const int HW = a.H * a.W, HoWo = a.Ho * a.Wo, KK = a.KH * a.KW;
  cd.y = cd.x = 0;
  if (IS_P) {
    const int stride = MODE == kFwd ? a.K : (MODE == kDx ? KK : HoWo);
    cd.lo = xx * stride;
    return cd;
  }
  if (MODE == kDw) {
    const int ci = fdiv(xx, a.dKK), kk = xx - ci * KK, kh = fdiv(kk, a.dKW), kw = kk - kh * a.KW;
    cd.y = kh * a.dh - a.ph;
    cd.x = kw * a.dw - a.pw;
    cd.lo = ci * HW + cd.y * a.W + cd.x;
    return cd;
  }
  const int b = MODE == kFwd ? fdiv(xx, a.dHoWo) : fdiv(xx, a.dHW);
  const int r = xx - b * (MODE == kFwd ? HoWo : HW);
  const int y = MODE == kFwd ? fdiv(r, a.dWo) : fdiv(r, a.dW);
  const int xc = r - y * (MODE == kFwd ? a.Wo : a.W);
  if (MODE == kFwd) {
    cd.y = y * a.sh - a.ph;
    cd.x = xc * a.sw - a.pw;
    cd.lo = b * a.Cin * HW + cd.y * a.W + cd.x;
  } else {
    cd.y = y + a.ph;
    cd.x = xc + a.pw;
    // stride 1: the gathered dY row is affine in (t1, t2); otherwise the
    // offset is formed per row (kx_src_strided)
    cd.lo = b * a.Cout * HoWo + ((a.sh == 1 && a.sw == 1) ? cd.y * a.Wo + cd.x : 0);
  }
  return cd;
}

// Wave-uniform part of row k = (t0, t1, t2) (flat k for the forward's P).
template <int MODE, bool IS_P>
WXX_HD int kx_uoff(const ConvArgs& a, int k, int t0, int t1, int t2) {
  const int HW = a.H * a.W, HoWo = a.Ho * a.Wo, KK = a.KH * a.KW;
  if (IS_P) {
    if (MODE == kFwd) return k;
    if (MODE == kDx) return t0 * a.Cin * KK + t1 * a.KW + t2;
    return t0 * a.Cout * HoWo + t1 * a.Wo + t2;
  }
  if (MODE == kFwd) return t0 * HW + t1 * a.dh * a.W + t2 * a.dw;
  if (MODE == kDx) return t0 * HoWo - t1 * a.dh * a.Wo - t2 * a.dw;  // stride 1
  return t0 * a.Cin * HW + t1 * a.sh * a.W + t2 * a.sw;
}

// Does column cd read memory in row (t1, t2)?  (dX with stride > 1 goes
// through kx_src_strided instead.)
template <int MODE, bool IS_P>
WXX_HD bool kx_valid(const ConvArgs& a, const KxCol& cd, int t1, int t2) {
  if (IS_P) return cd.ok;
  if (MODE == kFwd)
    return cd.ok && (unsigned)(cd.y + t1 * a.dh) < (unsigned)a.H &&
           (unsigned)(cd.x + t2 * a.dw) < (unsigned)a.W;
  if (MODE == kDx)
    return cd.ok && (unsigned)(cd.y - t1 * a.dh) < (unsigned)a.Ho &&
           (unsigned)(cd.x - t2 * a.dw) < (unsigned)a.Wo;
  return cd.ok && (unsigned)(t1 * a.sh + cd.y) < (unsigned)a.H &&
         (unsigned)(t2 * a.sw + cd.x) < (unsigned)a.W;
}

// dX's Q with a stride > 1: the dY position is (ih + ph - kh dh) / sh where
// that divides exactly.
WXX_HD bool kx_src_strided(const ConvArgs& a, const KxCol& cd, int t0, int t1, int t2, int& off) {
  const int th = cd.y - t1 * a.dh, tw = cd.x - t2 * a.dw;
  if (!cd.ok || th < 0 || tw < 0) return false;
  const int oh = fdiv(th, a.dsh), ow = fdiv(tw, a.dsw);
  if (oh * a.sh != th || ow * a.sw != tw || oh >= a.Ho || ow >= a.Wo) return false;
  off = cd.lo + t0 * a.Ho * a.Wo + oh * a.Wo + ow;
  return true;
}

// Source offset of row k = (t0, t1, t2) in column cd; false where zero.
template <int MODE, bool IS_P>
WXX_HD bool kx_src(const ConvArgs& a, const KxCol& cd, int k, int t0, int t1, int t2,
                   long long& off) {
  if (MODE == kDx && !IS_P && (a.sh != 1 || a.sw != 1)) {
    int o = 0;
    if (!kx_src_strided(a, cd, t0, t1, t2, o)) return false;
    off = o;
    return true;
  }
  if (!kx_valid<MODE, IS_P>(a, cd, t1, t2)) return false;
  off = (long long)cd.lo + kx_uoff<MODE, IS_P>(a, k, t0, t1, t2);
  return true;
}

// ---- layout choice ----------------------------------------------------------
// Distinct 128-byte lines (element offsets from a line-aligned base; all
// zero-loads count as one line) summed over the wave loads of one chunk
// of the tile starting at x0, for chunk kbase.
template <int MODE, bool IS_P, int BK>
inline long long conv_lines(const ConvArgs& a, bool xk, int x0, int kbase) {
  const int kend = a.K;
  long long total = 0;
  long long lines[64];
  auto count = [&](int n) {
    int distinct = 0;
    for (int i = 0; i < n; ++i) {
      bool seen = false;
      for (int j = 0; j < i; ++j) seen = seen || lines[j] == lines[i];
      distinct += !seen;
    }
    return distinct;
  };
  const int R1 = conv_r1(MODE, a), R2 = conv_r2(MODE, a);
  if (xk) {
    const XkUniform u = xk_uniform(MODE, a, kbase);
    for (int q = 0; q < Xk<BK>::kInst; ++q) {
      for (int l = 0; l < 64; ++l) {
        const XkSlot s = xk_slot<MODE, IS_P, BK>(a, x0, 64 * q + l);
        int off = 0;
        lines[l] = xk_src<MODE, IS_P>(a, s, u, kbase, kend - kbase, off) ? ((long long)off * 4) >> 7
                                                                          : -1;
      }
      total += count(64);
    }
  } else {
    for (int r = 0; r < BK; ++r) {
      const int k = kbase + r;
      const int t0 = k / (R1 * R2), t1 = (k - t0 * R1 * R2) / R2, t2 = k - (t0 * R1 + t1) * R2;
      for (int l = 0; l < 64; ++l) {
        const KxCol cd = kx_col<MODE, IS_P>(a, x0 + l);
        long long off = 0;
        lines[l] = k < kend && kx_src<MODE, IS_P>(a, cd, k, t0, t1, t2, off) ? (off * 4) >> 7 : -1;
      }
      total += count(64);
    }
  }
  return total;
}

}  // namespace wxx_conv
