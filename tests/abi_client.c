/* A plain C client of libkla_hip.so, built by tests/test_abi_c_client.py with a
 * C compiler against include/kla_hip.h alone: the boundary is a C ABI (no C++
 * or torch types). It makes only calls that need no GPU -- the version, a
 * workspace size, argument checks that fail before any HIP call, and an empty
 * problem -- and exits 0 when every result is the documented one.
 * argv[1]: the ABI version the Python binding expects. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "kla_hip.h"

static int fails = 0;

static void expect(int ok, const char *what) {
  if (!ok) {
    fprintf(stderr, "FAIL: %s\n", what);
    ++fails;
  }
}

int main(int argc, char **argv) {
  const int want_abi = argc > 1 ? atoi(argv[1]) : -1;
  expect(kla_hip_abi_version() == want_abi, "kla_hip_abi_version matches the binding's");

  /* The headline workspace: header plus records, a positive multiple of 8 bytes. */
  const size_t ws = kla_scan_workspace_bytes(KLA_SCAN_MOBIUS_FWD, 8, 4096, 2048);
  expect(ws > 256 && ws % 8 == 0, "kla_scan_workspace_bytes of the headline shape");

  /* A NULL input is rejected before any HIP call, with a message. */
  float *fake = (float *)(uintptr_t)0x7F0000000000ull; /* never dereferenced */
  int rc = kla_mobius_scan_fwd(NULL, fake, fake, NULL, NULL, fake, 2, 5, 7, fake, ws, NULL);
  expect(rc == KLA_ERR_INVALID_ARG, "NULL A gives KLA_ERR_INVALID_ARG");
  expect(strlen(kla_hip_last_error()) > 0, "the error has a message");

  /* A negative shape is rejected too. */
  rc = kla_affine_scan_fwd(KLA_DTYPE_F32, fake, fake, NULL, fake, -1, 5, 7, fake, ws, NULL);
  expect(rc == KLA_ERR_INVALID_ARG, "negative batch gives KLA_ERR_INVALID_ARG");

  /* An empty problem succeeds without launching anything. */
  rc = kla_mobius_scan_fwd(NULL, NULL, NULL, NULL, NULL, NULL, 0, 5, 7, NULL, 0, NULL);
  expect(rc == KLA_OK, "an empty problem is KLA_OK");

  if (fails == 0) printf("abi client ok (ABI %d, headline workspace %zu bytes)\n", kla_hip_abi_version(), ws);
  return fails == 0 ? 0 : 1;
}
