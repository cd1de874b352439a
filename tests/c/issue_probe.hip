// issue_probe -- what one wave64 pays per instruction on this GPU: the cost
// model behind the single-row space-saving chain (the longest row's stream
// is one wave's dependent sequence, so its time is the sum of these).
//
//   issue_probe [ITERS]
//
// One workgroup of one wave runs a loop of ITERS iterations (default 20000)
// of one instruction group, timed with s_memtime (the shader clock); the
// program prints the cycles per iteration and per group member.  Groups:
//   valu_dep    32 dependent v_add_u32
//   valu_indep  32 v_add_u32 over four independent registers
//   salu_dep    32 dependent s_add_u32
//   salu_indep  32 s_add_u32 over four independent registers
//   mixed       16 v_add_u32 and 16 s_add_u32, interleaved, independent
//   cndmask     32 dependent v_cndmask_b32 on an SGPR mask
//   dpp_min     8 dependent v_min_u32 DPP (quad_perm) with s_nop 1 between
//               (the two wait states a DPP read of the previous result needs)
//   readlane_rt 8 x (v_readlane to an SGPR, s_nop 3, s_add on it, v_add from it)
//   lane_sel    8 x (s_and, v_readlane with that SGPR as the lane select,
//               s_nop 3), each depending on the last through the SGPR
//   cmp_branch  8 x (v_cmp to an SGPR pair, s_cmp on it, s_cbranch not taken)
//   branch      8 taken s_branch to the next instruction
//   writelane   8 v_writelane_b32 with the lane select in M0
// Each group touches registers only (no memory inside the timed loop), and
// every wait state the ISA requires between its instructions is written.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>

#define REP8(x) x x x x x x x x
#define REP32(x) REP8(x) REP8(x) REP8(x) REP8(x)

template <int T>
__global__ void __launch_bounds__(64) issue_probe(int iters, int32_t *out, long long *cyc) {
  int32_t v = threadIdx.x, v1 = 1, v2 = 2, v3 = 3;
  uint32_t s = 5, s1 = 7;
  const long long t0 = clock64();
  for (int it = 0; it < iters; ++it) {
    if constexpr (T == 0) {
      asm volatile(REP32("v_add_u32 %0, %0, %1\n\t") : "+v"(v) : "v"(v1));
    } else if constexpr (T == 1) {
      asm volatile(REP8("v_add_u32 %0, %0, %4\n\tv_add_u32 %1, %1, %4\n\t"
                        "v_add_u32 %2, %2, %4\n\tv_add_u32 %3, %3, %4\n\t")
                   : "+v"(v), "+v"(v1), "+v"(v2), "+v"(v3)
                   : "v"(7));
    } else if constexpr (T == 2) {
      asm volatile(REP32("s_add_u32 %0, %0, %1\n\t") : "+s"(s) : "s"(s1) : "scc");
    } else if constexpr (T == 3) {
      uint32_t a = 1, b = 2, c = 3, d = 4;
      asm volatile(REP8("s_add_u32 %0, %0, %4\n\ts_add_u32 %1, %1, %4\n\t"
                        "s_add_u32 %2, %2, %4\n\ts_add_u32 %3, %3, %4\n\t")
                   : "+s"(a), "+s"(b), "+s"(c), "+s"(d)
                   : "s"(s1)
                   : "scc");
      s += a + b + c + d;
    } else if constexpr (T == 4) {
      uint32_t a = 1;
      asm volatile(REP8("v_add_u32 %0, %0, %3\n\ts_add_u32 %2, %2, %4\n\t"
                        "v_add_u32 %1, %1, %3\n\ts_add_u32 %2, %2, %4\n\t")
                   : "+v"(v), "+v"(v1), "+s"(a)
                   : "v"(7), "s"(s1)
                   : "scc");
      s += a;
    } else if constexpr (T == 5) {
      const uint64_t m = 0x5555555555555555ull;
      asm volatile(REP32("v_cndmask_b32_e64 %0, %0, %1, %2\n\t") : "+v"(v) : "v"(v1), "s"(m));
    } else if constexpr (T == 6) {
      asm volatile(REP8("v_min_u32_dpp %0, %0, %0 quad_perm:[1,0,3,2] row_mask:0xf "
                        "bank_mask:0xf\n\ts_nop 1\n\t")
                   : "+v"(v));
    } else if constexpr (T == 7) {
      uint32_t t;
      asm volatile(REP8("v_readlane_b32 %1, %0, 5\n\ts_nop 3\n\ts_add_u32 %1, %1, 1\n\t"
                        "v_add_u32 %0, %1, %0\n\t")
                   : "+v"(v), "=&s"(t)
                   :
                   : "scc");
    } else if constexpr (T == 8) {
      asm volatile(REP8("s_and_b32 %1, %1, 63\n\tv_readlane_b32 %1, %0, %1\n\ts_nop 3\n\t")
                   : "+v"(v), "+s"(s)
                   :
                   : "scc");
    } else if constexpr (T == 9) {
      uint64_t m;
      asm volatile(REP8("v_cmp_eq_u32_e64 %1, %0, -1\n\ts_cmp_lg_u64 %1, 0\n\t"
                        "s_cbranch_scc1 2f\n\t") "2:\n\t"
                   : "+v"(v), "=&s"(m)
                   :
                   : "scc");
    } else if constexpr (T == 10) {
      asm volatile(REP8("s_branch 1f\n1:\n\t")::);
    } else if constexpr (T == 11) {
      uint32_t m0s;
      asm volatile("s_mov_b32 %1, m0\n\ts_mov_b32 m0, 3\n\ts_nop 0\n\t"
                   REP8("v_writelane_b32 %0, %2, m0\n\t") "s_mov_b32 m0, %1\n\t"
                   : "+v"(v), "=&s"(m0s)
                   : "s"(s));
    }
  }
  const long long t1 = clock64();
  out[threadIdx.x] = v + v1 + v2 + v3 + static_cast<int32_t>(s);
  if (threadIdx.x == 0) cyc[0] = t1 - t0;
}

#define CK(x)                                                                 \
  do {                                                                        \
    hipError_t e_ = (x);                                                      \
    if (e_ != hipSuccess) {                                                   \
      std::fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), \
                   __LINE__);                                                 \
      return 1;                                                               \
    }                                                                         \
  } while (0)

int main(int argc, char **argv) {
  const int iters = argc > 1 ? std::atoi(argv[1]) : 20000;
  if (iters < 1) {
    std::fprintf(stderr, "ITERS must be positive\n");
    return 1;
  }
  int32_t *out;
  long long *cyc;
  CK(hipMalloc(&out, 64 * sizeof(int32_t)));
  CK(hipMalloc(&cyc, sizeof(long long)));
  const char *names[] = {"valu_dep", "valu_indep", "salu_dep", "salu_indep",
                         "mixed", "cndmask", "dpp_min", "readlane_rt",
                         "lane_sel", "cmp_branch", "branch", "writelane"};
  const int members[] = {32, 32, 32, 32, 32, 32, 8, 8, 8, 8, 8, 8};
  for (int t = 0; t < 12; ++t) {
    long long c = 0;
    for (int rep = 0; rep < 3; ++rep) { // the third launch is reported
      switch (t) {
#define SP_CASE(T) \
  case T:          \
    issue_probe<T><<<1, 64>>>(iters, out, cyc); \
    break;
        SP_CASE(0) SP_CASE(1) SP_CASE(2) SP_CASE(3) SP_CASE(4) SP_CASE(5)
        SP_CASE(6) SP_CASE(7) SP_CASE(8) SP_CASE(9) SP_CASE(10) SP_CASE(11)
#undef SP_CASE
      }
      CK(hipGetLastError());
      CK(hipDeviceSynchronize());
      CK(hipMemcpy(&c, cyc, sizeof(c), hipMemcpyDeviceToHost));
    }
    std::printf("group=%s cycles_per_iter=%.1f cycles_per_member=%.2f\n", names[t],
                static_cast<double>(c) / iters, static_cast<double>(c) / iters / members[t]);
  }
  CK(hipFree(out));
  CK(hipFree(cyc));
  return 0;
}
