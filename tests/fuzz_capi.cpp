// Host-side fuzz of the C ABI argument validation and size arithmetic.  Many
// calls start from valid argument sets with fake device addresses, so the fuzz
// must only ever run where no GPU is visible: there, calls that pass
// validation fail at their first HIP call; with a device they would launch
// kernels on those addresses.  main() therefore refuses to run (exit code 3,
// "device visible") when the HIP runtime reports any device, and
// tests/test_capi_sanitizers.py hides every device from this process through
// its environment.  Built with AddressSanitizer and UndefinedBehaviorSanitizer
// on the host pass; prints "done" at the end.
#include <hip/hip_runtime_api.h>
#include <cstdio>
#include <cstdint>
#include <cstring>
#include <random>
#include "fsk_decode.h"

static std::mt19937_64 rng(12345);
static int64_t pick_i64() {
  static const int64_t v[] = {-1, 0, 1, 2, 7, 8, 15, 16, 17, 31, 32, 64, 128, 256, 1000, 4096, 65536,
                              (1LL << 31) - 1, -(1LL << 31), 1LL << 31, 1LL << 40, INT64_MAX, INT64_MIN};
  if (rng() % 4 == 0) return (int64_t)(rng() % 100000) - 50000;
  return v[rng() % (sizeof(v) / sizeof(v[0]))];
}
static int pick_i() { return (int)pick_i64(); }
static void* pick_p() {
  switch (rng() % 4) {
    case 0: return nullptr;
    case 1: return (void*)0x100000;
    case 2: return (void*)0x100004;
    default: return (void*)0x7f0000001000ULL;
  }
}
// Host lengths for the *_host entry points (host memory, read by the call).
static int32_t host_lens[65];
static const int32_t* pick_host_lens() {
  for (int i = 0; i < 65; ++i) host_lens[i] = rng() % 3 ? (int32_t)(rng() % 70000) : (int32_t)pick_i();
  return host_lens;
}
static void check(int st, const char* fn) {
  if (st > 0 || st < -4) { printf("%s returned %d\n", fn, st); }
  const char* e = fsk_last_error();
  if (!e) printf("%s: null last_error\n", fn);
  else (void)strlen(e);
}
int main() {
  int devices = 0;
  if (hipGetDeviceCount(&devices) == hipSuccess && devices > 0) {
    printf("device visible: the fuzz runs only where no GPU is visible\n");
    return 3;
  }
  for (int it = 0; it < 20000; ++it) {
    int64_t n = fsk_workspace_bytes(pick_i(), pick_i(), pick_i(), pick_i(), pick_i(), pick_i64(), pick_i(), pick_i());
    if (n < -4) printf("workspace_bytes %lld\n", (long long)n);
    (void)fsk_score_workspace_bytes(pick_i(), pick_i(), pick_i());
    check(fsk_decode_varlen(pick_p(), pick_i64(), pick_i64(), pick_p(), pick_i64(), pick_i64(), pick_p(), pick_i64(),
                            pick_i64(), (const int32_t*)pick_p(), pick_i64(), (const float*)pick_p(), pick_i(),
                            (const float*)pick_p(), (const float*)pick_p(), pick_p(), pick_i64(), pick_i64(),
                            pick_i(), pick_i(), pick_i(), pick_i(), pick_i() & 3, pick_i() & 3, pick_i() & 3, 0.1f,
                            pick_p(), pick_i64(), pick_i(), nullptr), "varlen");
    check(fsk_decode_paged(pick_p(), pick_i64(), pick_i64(), pick_p(), pick_i64(), pick_i64(), pick_i64(), pick_p(),
                           pick_i64(), pick_i64(), pick_i64(), (const int32_t*)pick_p(), pick_i64(), pick_i(),
                           (const int32_t*)pick_p(), pick_i(), pick_i(), (const float*)pick_p(), pick_i(),
                           (const float*)pick_p(), (const float*)pick_p(), pick_p(), pick_i64(), pick_i64(), pick_i(),
                           pick_i(), pick_i(), pick_i(), pick_i() & 3, pick_i() & 3, pick_i() & 3, 0.1f, pick_p(),
                           pick_i64(), pick_i(), nullptr), "paged");
    check(fsk_decode_varlen_host(pick_p(), pick_i64(), pick_i64(), pick_p(), pick_i64(), pick_i64(), pick_p(),
                                 pick_i64(), pick_i64(), pick_host_lens(), pick_i64(), (const float*)pick_p(), pick_i(),
                                 (const float*)pick_p(), (const float*)pick_p(), pick_p(), pick_i64(), pick_i64(),
                                 (int)(rng() % 70) - 2, pick_i(), pick_i(), pick_i(), pick_i() & 3, pick_i() & 3,
                                 pick_i() & 3, 0.1f, pick_p(), pick_i64(), pick_i(), nullptr), "varlen-host");
    check(fsk_decode_paged_host(pick_p(), pick_i64(), pick_i64(), pick_p(), pick_i64(), pick_i64(), pick_i64(),
                                pick_p(), pick_i64(), pick_i64(), pick_i64(), (const int32_t*)pick_p(), pick_i64(),
                                pick_i(), pick_host_lens(), pick_i(), pick_i(), (const float*)pick_p(), pick_i(),
                                (const float*)pick_p(), (const float*)pick_p(), pick_p(), pick_i64(), pick_i64(),
                                (int)(rng() % 70) - 2, pick_i(), pick_i(), pick_i(), pick_i() & 3, pick_i() & 3,
                                pick_i() & 3, 0.1f, pick_p(), pick_i64(), pick_i(), nullptr), "paged-host");
    check(fsk_decode_dense(pick_p(), pick_i64(), pick_i64(), pick_p(), pick_i64(), pick_i64(), pick_i64(), pick_p(),
                           pick_i64(), pick_i64(), pick_i64(), pick_i64(), (const int32_t*)pick_p(),
                           (const int32_t*)pick_p(), (const float*)pick_p(), pick_i(), (const float*)pick_p(),
                           (const float*)pick_p(), (const float*)pick_p(), pick_p(), pick_i64(), pick_i64(), pick_i(),
                           pick_i(), pick_i(), pick_i(), pick_i() & 3, pick_i() & 3, pick_i() & 3, 0.1f, pick_p(),
                           pick_i64(), pick_i(), nullptr), "dense");
    check(fsk_paged_write(pick_p(), pick_i64(), pick_i64(), pick_p(), pick_i64(), pick_i64(), (const int64_t*)pick_p(),
                          pick_i64(), pick_p(), pick_i64(), pick_i64(), pick_i64(), pick_p(), pick_i64(), pick_i64(),
                          pick_i64(), pick_i(), pick_i(), pick_i(), pick_i(), pick_i() & 3, pick_i() & 3,
                          (const float*)pick_p(), (const float*)pick_p(), (int32_t*)pick_p(), pick_i64(),
                          (const int64_t*)pick_p(), pick_i64(), nullptr), "write");
    check(fsk_set_option(rng() % 2 ? "xcd_skew" : "nope", pick_i64()), "set_option");
  }
  // Valid paged arguments with 1-3 fields perturbed (deeper validation paths).
  for (int it = 0; it < 200000; ++it) {
    int64_t a[37] = {0x100000, 32 * 128, 128, 0x200000, 8 * 16 * 128, 16 * 128, 128, 0x300000, 8 * 16 * 128,
                     16 * 128, 128, 0x400000, 64, 64, 0x500000, 100, 16, 0, 0, 0, 0, 0x600000, 32 * 128, 128,
                     4, 32, 8, 128, 0, 0, 0, 0, 0x700000, (int64_t)1 << 30, 0, 0, 0};
    const int nper = 1 + rng() % 3;
    for (int j = 0; j < nper; ++j) {
      const int f = rng() % 37;
      if (f == 31) continue;  // sm_scale slot (float)
      a[f] = (f == 0 || f == 3 || f == 7 || f == 11 || f == 14 || f == 17 || f == 19 || f == 20 || f == 21 ||
              f == 32 || f == 36) ? (int64_t)(uintptr_t)pick_p() : pick_i64();
    }
    check(fsk_decode_paged((void*)a[0], a[1], a[2], (void*)a[3], a[4], a[5], a[6], (void*)a[7], a[8], a[9], a[10],
                           (const int32_t*)a[11], a[12], (int)a[13], (const int32_t*)a[14], (int)a[15], (int)a[16],
                           (const float*)a[17], (int)a[18], (const float*)a[19], (const float*)a[20], (void*)a[21],
                           a[22], a[23], (int)a[24], (int)a[25], (int)a[26], (int)a[27], (int)a[28], (int)a[29],
                           (int)a[30], 0.088f, (void*)a[32], a[33], (int)a[34], nullptr), "paged-perturbed");
    // the same arguments with host lengths (valid host memory, random values)
    if ((int)a[24] >= 0 && (int)a[24] <= 65)
      check(fsk_decode_paged_host((void*)a[0], a[1], a[2], (void*)a[3], a[4], a[5], a[6], (void*)a[7], a[8], a[9],
                                  a[10], (const int32_t*)a[11], a[12], (int)a[13], pick_host_lens(), (int)a[15],
                                  (int)a[16], (const float*)a[17], (int)a[18], (const float*)a[19],
                                  (const float*)a[20], (void*)a[21], a[22], a[23], (int)a[24], (int)a[25],
                                  (int)a[26], (int)a[27], (int)a[28], (int)a[29], (int)a[30], 0.088f, (void*)a[32],
                                  a[33], (int)a[34], nullptr), "paged-host-perturbed");
    (void)fsk_workspace_bytes((int)(rng() % 4), (int)a[24], (int)a[25], (int)a[26], (int)a[27], (a[13] & 0xFFFFFF) * 16,
                              (int)a[16], (int)a[34]);
  }
  // Valid write arguments with 1-3 fields perturbed.
  for (int it = 0; it < 200000; ++it) {
    int64_t a[29] = {0x100000, 8 * 128, 128, 0x200000, 8 * 128, 128, 0x300000, 64, 0x400000, 8 * 16 * 128, 16 * 128,
                     128, 0x500000, 8 * 16 * 128, 16 * 128, 128, 100, 16, 8, 128, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    const int nper = 1 + rng() % 3;
    for (int j = 0; j < nper; ++j) {
      const int f = rng() % 29;
      a[f] = (f == 0 || f == 3 || f == 6 || f == 8 || f == 12 || f == 22 || f == 23 || f == 24 || f == 26)
                 ? (int64_t)(uintptr_t)pick_p() : pick_i64();
    }
    check(fsk_paged_write((void*)a[0], a[1], a[2], (void*)a[3], a[4], a[5], (const int64_t*)a[6], a[7], (void*)a[8],
                          a[9], a[10], a[11], (void*)a[12], a[13], a[14], a[15], (int)a[16], (int)a[17], (int)a[18],
                          (int)a[19], (int)a[20], (int)a[21], (const float*)a[22], (const float*)a[23],
                          (int32_t*)a[24], a[25], (const int64_t*)a[26], a[27], nullptr), "write-perturbed");
  }
  for (int it = 0; it < 100000; ++it) {
    int64_t a[16] = {0x100000, 8 * 16 * 128, 16 * 128, 128, 0x200000, 64, 64, 0x300000, 100, 16, 4, 8, 128, 0,
                     0x400000, 0};
    const int nper = 1 + rng() % 3;
    for (int j = 0; j < nper; ++j) {
      const int f = rng() % 16;
      a[f] = (f == 0 || f == 4 || f == 7 || f == 14) ? (int64_t)(uintptr_t)pick_p() : pick_i64();
    }
    check(fsk_paged_gather((void*)a[0], a[1], a[2], a[3], (const int32_t*)a[4], a[5], (int)a[6], (const int32_t*)a[7],
                           (int)a[8], (int)a[9], (int)a[10], (int)a[11], (int)a[12], (int)a[13], (void*)a[14],
                           nullptr), "gather-perturbed");
  }
  fsk_set_option("xcd_skew", 3);
  printf("done\n");
  return 0;
}
