/*
 * backend.c — backend factory with BACKEND_HIP (the reference's
 * backend.c:5-66 with the HIP kind added): AUTO tries HIP, then CPU;
 * an explicit HIP request returns NULL when no device (or no HIP build) is
 * available, as the reference does for CUDA (backend.c:27-33).
 */
#include "backend_internal.h"

#include <stdlib.h>

Backend *backend_create(const BackendConfig *cfg) {
  BackendConfig local = {0};
  if (cfg) {
    local = *cfg;
  } else {
    local.kind = BACKEND_AUTO;
    local.threads = 1;
  }
  if (local.kind == BACKEND_AUTO) {
#if defined(USE_HIP) && USE_HIP == 1
    BackendConfig h = local;
    h.kind = BACKEND_HIP;
    Backend *b = backend_hip_create(&h);
    if (b) return b;
#endif
    local.kind = BACKEND_CPU;
    return backend_cpu_create(&local);
  }
  if (local.kind == BACKEND_HIP) {
#if defined(USE_HIP) && USE_HIP == 1
    return backend_hip_create(&local);
#else
    return NULL;
#endif
  }
  if (local.kind == BACKEND_CUDA) return NULL; /* not part of this build */
  return backend_cpu_create(&local);
}

void backend_destroy(Backend *b) {
  if (!b) return;
#if defined(USE_HIP) && USE_HIP == 1
  if (b->cfg.kind == BACKEND_HIP) {
    backend_hip_destroy(b);
    return;
  }
#endif
  backend_cpu_destroy(b);
}

const KernelVTable *backend_kernels(const Backend *b) { return b ? &b->kernels : NULL; }

BackendKind backend_kind(const Backend *b) { return b ? b->cfg.kind : BACKEND_CPU; }

BackendConfig backend_config(const Backend *b) {
  BackendConfig c = {0};
  if (b) c = b->cfg;
  return c;
}
