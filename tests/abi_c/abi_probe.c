/* The header as plain C11 (and, compiled again by g++, as C++17), linked against the
 * library: host-only entry points, no GPU needed. Prints "ok" on success. */
#include <stdio.h>
#include <string.h>

#include "exl3_moe.h"

int main(void) {
  if (exl3_abi_version() <= 0) return 1;
  exl3_tuning t;
  if (exl3_get_tuning(&t) != EXL3_OK) return 2;
  if (exl3_set_tuning(&t) != EXL3_OK) return 3;
  if (t.weight_form != EXL3_FORM_REFERENCE) return 6;
  t.weight_form = 7;
  if (exl3_set_tuning(&t) != EXL3_ERR_INVALID) return 7;
  exl3_trellis_desc d;
  memset(&d, 0, sizeof d);
  d.trellis = (const void *)0x1000;
  d.in_features = 100; /* not a multiple of 128 */
  d.out_features = 128;
  d.K = 4;
  d.codebook = EXL3_CB_MCG;
  exl3_path_info info;
  if (exl3_trellis_path_info(&d, 1, &info) != EXL3_ERR_INVALID) return 4;
  if (!exl3_last_error() || !exl3_last_error()[0]) return 5;
  printf("ok\n");
  return 0;
}
