// Host build of the device arithmetic shared by the gfx950 kernels (csrc/geometry_math.h: Wigner-D
// coefficients, their closed-form VJP and the envelope; csrc/nl_math.h: the neighbour-list
// distance predicates and cap keys), for the CPU tests in tests/test_host_math.py.  Built by that
// test with g++ under AddressSanitizer and UndefinedBehaviorSanitizer and -ffp-contract=off (the
// device build's contract(off) pragma).  Test infrastructure only; nothing here ships.
//
//   host_math <mode> <n> <param> <input.bin> <output.bin>
// modes (all arrays little-endian fp32 unless noted):
//   wigner   in: jd[35], ev[n][3]                 out: coef[n][35]        (param = gamma)
//   vjp      in: jd[35], ev[n][3], g_coef[n][35]  out: g_ev[n][3]         (param = gamma)
//   envelope in: d[n]                             out: env[n], denv[n]    (param = cutoff)
//   nl       in: a[n][3], b[n][3], sh[n][3]       out: norm2_fma(a, b)[n], sum_sq(a - b)[n],
//                                                      disp2(a, b, sh)[n], cap_d2(a, b, sh)[n]
//   key      in: d1[n] f32, a1[n] i32, c1[n] i32, d2[n] f32, a2[n] i32, c2[n] i32
//            out: key_le[n] i32, key_lt[n] i32
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "geometry_math.h"
#include "nl_math.h"

namespace {

std::vector<char> slurp(const char* path) {
  std::vector<char> b;
  FILE* f = std::fopen(path, "rb");
  if (!f) return b;
  char buf[1 << 16];
  size_t k;
  while ((k = std::fread(buf, 1, sizeof buf, f)) > 0) b.insert(b.end(), buf, buf + k);
  std::fclose(f);
  return b;
}

// Reads `count` 4-byte values at *off, advancing it; false if the input is too short.
template <class T>
bool take(const std::vector<char>& in, size_t* off, size_t count, std::vector<T>* out) {
  static_assert(sizeof(T) == 4, "4-byte elements");
  if (*off + count * 4 > in.size()) return false;
  out->resize(count);
  if (count) std::memcpy(out->data(), in.data() + *off, count * 4);
  *off += count * 4;
  return true;
}

int fail(const char* what) {
  std::fprintf(stderr, "host_math: %s\n", what);
  return 2;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 6) return fail("usage: host_math <mode> <n> <param> <in> <out>");
  const char* mode = argv[1];
  const long n = std::strtol(argv[2], nullptr, 10);
  const float param = std::strtof(argv[3], nullptr);
  if (n < 0 || n > (1L << 24)) return fail("bad n");
  const std::vector<char> in = slurp(argv[4]);
  size_t off = 0;
  std::vector<float> out;
  std::vector<int32_t> iout;
  if (!std::strcmp(mode, "wigner") || !std::strcmp(mode, "vjp")) {
    const bool vjp = mode[0] == 'v';
    std::vector<float> jd, ev, gc;
    if (!take(in, &off, 35, &jd) || !take(in, &off, 3 * n, &ev) ||
        (vjp && !take(in, &off, 35 * n, &gc)))
      return fail("short input");
    out.assign((vjp ? 3 : 35) * n, 0.f);
    for (long e = 0; e < n; ++e) {
      if (vjp)
        tta_geo::wigner_vjp(&ev[3 * e], param, jd.data(), &gc[35 * e], &out[3 * e]);
      else
        tta_geo::wigner_coef(&ev[3 * e], param, jd.data(), &out[35 * e]);
    }
  } else if (!std::strcmp(mode, "envelope")) {
    std::vector<float> d;
    if (!take(in, &off, n, &d)) return fail("short input");
    out.resize(2 * n);
    for (long e = 0; e < n; ++e) {
      out[e] = tta_geo::envelope(d[e], param);
      out[n + e] = tta_geo::envelope_grad(d[e], param);
    }
  } else if (!std::strcmp(mode, "nl")) {
    std::vector<float> a, b, sh;
    if (!take(in, &off, 3 * n, &a) || !take(in, &off, 3 * n, &b) || !take(in, &off, 3 * n, &sh))
      return fail("short input");
    out.resize(4 * n);
    for (long e = 0; e < n; ++e) {
      const float3 pa = tta_nl::ld3(a.data(), (int)e), pb = tta_nl::ld3(b.data(), (int)e);
      const float3 ps = tta_nl::ld3(sh.data(), (int)e);
      out[e] = tta_nl::norm2_fma(pa, pb);
      out[n + e] = tta_nl::sum_sq(tta_nl::rn_sub(pa.x, pb.x), tta_nl::rn_sub(pa.y, pb.y),
                                  tta_nl::rn_sub(pa.z, pb.z));
      out[2 * n + e] = tta_nl::disp2(pa, pb, ps);
      out[3 * n + e] = tta_nl::cap_d2(pa, pb, ps);
    }
  } else if (!std::strcmp(mode, "key")) {
    std::vector<float> d1, d2;
    std::vector<int32_t> a1, c1, a2, c2;
    if (!take(in, &off, n, &d1) || !take(in, &off, n, &a1) || !take(in, &off, n, &c1) ||
        !take(in, &off, n, &d2) || !take(in, &off, n, &a2) || !take(in, &off, n, &c2))
      return fail("short input");
    iout.resize(2 * n);
    for (long e = 0; e < n; ++e) {
      iout[e] = tta_nl::key_le(d1[e], a1[e], c1[e], d2[e], a2[e], c2[e]);
      iout[n + e] = tta_nl::key_lt(d1[e], a1[e], c1[e], d2[e], a2[e], c2[e]);
    }
  } else {
    return fail("unknown mode");
  }
  if (off != in.size()) return fail("input longer than the mode reads");
  FILE* f = std::fopen(argv[5], "wb");
  if (!f) return fail("cannot write output");
  const size_t bytes = out.empty() ? iout.size() * 4 : out.size() * 4;
  const void* src = out.empty() ? static_cast<const void*>(iout.data())
                                : static_cast<const void*>(out.data());
  const bool ok = bytes == 0 || std::fwrite(src, 1, bytes, f) == bytes;
  std::fclose(f);
  return ok ? 0 : fail("short write");
}
