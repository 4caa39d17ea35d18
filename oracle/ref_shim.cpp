// C-ABI binding of the reference's own EXL3 codec, compiled from the source
// files where they lie under the reference checkout (never copied here) into
// oracle/_ref/libexl3ref.so. Test infrastructure only: it is the second
// opinion the CPU oracle (exl3_oracle.c) is checked against, and the source of
// the golden fixtures under tests/golden/.
//
// Binds: exl3::codebook_value (exl3.h:41), exl3::decode_inner (exl3.h:44),
// exl3::reconstruct (exl3.h:48).
#include <cstdint>

#include "exl3.h"

extern "C" {

void ref_codebook_lut(int cb, uint16_t* out) {
  for (uint32_t s = 0; s < 65536u; ++s)
    out[s] = exl3::codebook_value((uint16_t)s, (exl3::Codebook)cb);
}

static exl3::Exl3Tensor ref_tensor(const uint16_t* trellis, int64_t in, int64_t out, int K, int cb,
                                   const uint16_t* suh, const uint16_t* svh) {
  exl3::Exl3Tensor t;
  t.trellis = trellis;
  t.K = K;
  t.codebook = (exl3::Codebook)cb;
  t.in_features = in;
  t.out_features = out;
  t.suh = suh;
  t.svh = svh;
  return t;
}

// Geometry is validated here so the reference's abort() paths are never hit.
int ref_decode_inner(const uint16_t* trellis, int64_t in, int64_t out, int K, int cb, uint16_t* w,
                     int threads) {
  if (in <= 0 || out <= 0 || in % 16 || out % 16 || K < 1 || K > 8 || cb < 0 || cb > 2) return -1;
  exl3::decode_inner(ref_tensor(trellis, in, out, K, cb, nullptr, nullptr), w, threads);
  return 0;
}

int ref_reconstruct(const uint16_t* trellis, int64_t in, int64_t out, int K, int cb,
                    const uint16_t* suh, const uint16_t* svh, uint16_t* w, int threads) {
  if (in <= 0 || out <= 0 || in % 128 || out % 128 || K < 1 || K > 8 || cb < 0 || cb > 2) return -1;
  exl3::reconstruct(ref_tensor(trellis, in, out, K, cb, suh, svh), w, threads);
  return 0;
}

}  // extern "C"
