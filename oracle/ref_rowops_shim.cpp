// TEST INFRASTRUCTURE ONLY: a C entry point over the reference's own row-ops oracle
// (kernels/rowops_rtl/tb/verilator/rowops_ref.h, compiled in place from the reference
// checkout by oracle/Makefile).  The four regions a, b, c, p are laid out at fixed
// 2^40-apart addresses of one flat address space; the job's writes land in `c`.
#include <cstdint>
#include <cstring>

#include "rowops_ref.h"

namespace {
constexpr uint64_t kA = 1ull << 40, kB = 2ull << 40, kC = 3ull << 40, kP = 4ull << 40;
struct Regions {
  const uint8_t *a, *b, *p;
  uint8_t* c;
  uint64_t na, nb, nc, np;
};
ro::PState g_ps;
}  // namespace

extern "C" int ref_rowops(const uint8_t* a, uint64_t na, const uint8_t* b, uint64_t nb, uint8_t* c,
                          uint64_t nc, const uint8_t* p, uint64_t np, uint32_t op, uint32_t n,
                          uint32_t c1, uint32_t c2, uint32_t a_s1, uint32_t a_s2, uint32_t b_s1,
                          uint32_t b_s2, uint32_t c_s1, uint32_t c_s2, long long eps, uint32_t aux,
                          uint32_t bq_sh, uint32_t win_lo, uint32_t win_hi) {
  Regions r{a, b, p, c, na, nb, nc, np};
  ro::Mem m{[&r](uint64_t addr) -> uint8_t {
    auto in = [&](uint64_t base, const uint8_t* ptr, uint64_t len) -> int {
      return addr >= base && addr < base + len && ptr ? (int)ptr[addr - base] : -1;
    };
    int v;
    if ((v = in(kA, r.a, r.na)) >= 0) return (uint8_t)v;
    if ((v = in(kB, r.b, r.nb)) >= 0) return (uint8_t)v;
    if ((v = in(kC, r.c, r.nc)) >= 0) return (uint8_t)v;
    if ((v = in(kP, r.p, r.np)) >= 0) return (uint8_t)v;
    return 0;
  }};
  ro::Job j;
  j.op = op; j.n = n; j.c1 = c1; j.c2 = c2;
  j.a = kA; j.b = kB; j.c = kC; j.p = kP;
  j.a_s1 = a_s1; j.a_s2 = a_s2; j.b_s1 = b_s1; j.b_s2 = b_s2; j.c_s1 = c_s1; j.c_s2 = c_s2;
  j.eps = (uint64_t)eps; j.aux = aux; j.bq_sh = bq_sh; j.win_lo = win_lo; j.win_hi = win_hi;
  auto writes = ro::run(j, m, &g_ps);
  for (const auto& w : writes) {
    if (w.addr < kC || w.addr + w.bytes.size() > kC + nc) return -1;   // outside c
    std::memcpy(c + (w.addr - kC), w.bytes.data(), w.bytes.size());
  }
  return 0;
}

extern "C" void ref_rowops_reset() { g_ps = ro::PState(); }

extern "C" int ref_rowops_table_image(uint8_t* out) {
  auto img = ro::table_image();
  std::memcpy(out, img.data(), img.size());
  return 0;
}
