// Host-only check of launch_nt's argument guards: every case below must be refused with
// hipErrorInvalidValue before the launcher touches the device (no GPU is needed, none is used).
// Built and run by tests/test_abi.py::test_launch_nt_refuses_mismatched_addend_alias.
#include <stdio.h>

#include "../../dmuon_amd/csrc/dmuon_amd_internal.h"

using dmuon::NtArgs;

static NtArgs square(uint16_t* buf, int M, int K, int N) {
  NtArgs a{};
  a.A = buf; a.lda = K; a.sA = 0;
  a.B = buf; a.ldb = K; a.sB = 0;
  a.M = M; a.N = N; a.K = K; a.L = 1;
  a.mt = M / 256; a.nt = N / 256; a.tiles_per_mat = a.mt * a.nt; a.tri = 0;
  a.mode = dmuon::EPI_SYM;
  a.C = buf; a.ldc = N; a.sC = 0;
  a.D = buf + 1; a.ldd = N; a.sD = 0;
  return a;
}

int main() {
  static uint16_t buf[64];   // never dereferenced: every case is refused on the host
  int bad = 0;
  auto expect_refused = [&](const char* what, const NtArgs& a) {
    const hipError_t e = dmuon::launch_nt(a, 256, nullptr);
    printf("%-58s -> %s\n", what, e == hipErrorInvalidValue ? "refused" : "NOT REFUSED");
    if (e != hipErrorInvalidValue) ++bad;
  };
  // the probe fault's shape: C named as A (C_IS_A) while A is a 4096 x 64 panel and the
  // epilogue would read C as 4096 x 4096
  NtArgs a = square(buf, 4096, 64, 4096);
  a.c_in = dmuon::C_IS_A;
  expect_refused("C_IS_A, K=64 != M=4096", a);
  a = square(buf, 512, 512, 512);
  a.c_in = dmuon::C_IS_A;
  a.C = buf + 8;
  expect_refused("C_IS_A, C != A", a);
  a = square(buf, 512, 512, 512);
  a.c_in = dmuon::C_IS_A;
  a.ldc = 1024;
  expect_refused("C_IS_A, ldc != lda", a);
  a = square(buf, 512, 512, 512);
  a.c_in = dmuon::C_IS_A;
  a.L = 2; a.sA = 512 * 512; a.sB = a.sA; a.sC = 0;
  expect_refused("C_IS_A, batch stride of C != A's", a);
  a = square(buf, 512, 512, 1024);
  a.c_in = dmuon::C_IS_A;
  expect_refused("C_IS_A, N=1024 != M=512", a);
  a = square(buf, 4096, 64, 4096);
  a.c_in = dmuon::C_IS_B;
  expect_refused("C_IS_B, K=64 != M=4096", a);
  a = square(buf, 512, 512, 512);
  a.c_in = dmuon::C_IS_B;
  a.C = buf + 8;
  expect_refused("C_IS_B, C != B", a);
  a = square(buf, 512, 512, 512);
  a.c_in = 7;
  expect_refused("unknown c_in code", a);
  // the K loop may stop short of K only at a slice boundary inside the operands
  a = square(buf, 512, 512, 512);
  a.k_loop = 576;
  expect_refused("k_loop=576 > K=512", a);
  a = square(buf, 512, 512, 512);
  a.k_loop = 480;
  expect_refused("k_loop=480 not a multiple of 64", a);
  a = square(buf, 512, 512, 512);
  a.k_loop = -64;
  expect_refused("k_loop < 0", a);
  // unread padding starts at a slice boundary, at the same place for both sides of a triangle
  a = square(buf, 512, 512, 512);
  a.live_rows = 448 + 32;
  expect_refused("live_rows not a multiple of 64", a);
  a = square(buf, 512, 512, 512);
  a.live_cols = -64;
  expect_refused("live_cols < 0", a);
  a = square(buf, 512, 512, 512);
  a.tri = 1;
  a.live_rows = 448;
  a.live_cols = 384;
  expect_refused("triangle with live_rows != live_cols", a);
  // the block -> logical tile map of the NT kernels is a permutation of the launch's tiles
  // (a tile computed twice, or one past the launch, would be a wrong result or an out-of-bounds
  // access): launch sizes 1 .. 4096 and the c4 / c5 launch sizes
  int map_bad = 0;
  static int seen[1 << 16];
  const int sizes[] = {2688, 4352, 4608, 6144, 8704, 16384, 28672, 57344};
  for (int k = 0; k < 4096 + 8 && !map_bad; ++k) {
    const int nb = k < 4096 ? k + 1 : sizes[k - 4096];
    for (int t = 0; t < nb; ++t) seen[t] = 0;
    for (int b = 0; b < nb; ++b) {
      const int t = dmuon::nt_block_tile(b, nb);
      if (t < 0 || t >= nb || seen[t]++) {
        printf("block %d of %d maps to tile %d: not a permutation\n", b, nb, t);
        map_bad = 1;
        break;
      }
    }
  }
  printf("block -> tile map: %s\n", map_bad ? "NOT A PERMUTATION" : "permutation for every size");
  if (bad || map_bad) {
    if (bad) printf("%d case(s) not refused\n", bad);
    return 1;
  }
  printf("all refused\n");
  return 0;
}
