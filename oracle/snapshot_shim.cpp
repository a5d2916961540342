// snapshot_shim.cpp -- test harness around the reference's snapshot I/O.
//
// TEST INFRASTRUCTURE ONLY.  Compiled together with the reference's
// replay/session_snapshot.cpp, read in place from /root/reference (see
// oracle/Makefile), into oracle/_ref/libsnapshot_ref.so.  It exposes the
// reference's own SessionSnapshot::load and ::save through plain C entry
// points so tests can check that files written by this library load in the
// reference and round-trip to the same bytes.  SessionSnapshot::capture needs
// the reference's V2 RuntimeContext, which is not built; the library is
// opened with lazy binding and capture is never called.
#include "replay/session_snapshot.h"

#include <cstdio>
#include <exception>
#include <new>

using adaptq::SessionSnapshot;

extern "C" {

// Returns a handle, or NULL with the reference's exception text in err.
void *snapref_load(const char *path, char *err, int err_len) {
  try {
    return new SessionSnapshot(SessionSnapshot::load(path));
  } catch (const std::exception &e) {
    std::snprintf(err, (size_t)err_len, "%s", e.what());
    return nullptr;
  }
}

void snapref_free(void *s) { delete static_cast<SessionSnapshot *>(s); }

// n_layers, n_heads, dim, bits, n_tokens, heads in the file, flags
void snapref_info(void *s, int *out) {
  const SessionSnapshot *p = static_cast<SessionSnapshot *>(s);
  out[0] = p->n_layers();
  out[1] = p->n_heads();
  out[2] = p->dim();
  out[3] = p->bits();
  out[4] = p->n_tokens();
  out[5] = (int)p->heads().size();
  out[6] = (p->has_token_log() ? 1 : 0) | (p->has_strategy_state() ? 2 : 0);
}

// Head block i: coordinates and sizes in ints[4], pointers to its arrays.
int snapref_head(void *s, int i, int *ints, const unsigned char **data, const float **scales,
                 const unsigned char **tags) {
  const SessionSnapshot *p = static_cast<SessionSnapshot *>(s);
  if (i < 0 || i >= (int)p->heads().size()) return -1;
  const auto &h = p->heads()[(size_t)i];
  ints[0] = h.layer;
  ints[1] = h.head;
  ints[2] = h.cache_size;
  ints[3] = h.slot_bytes;
  *data = h.storage_data.data();
  *scales = h.scales.data();
  *tags = h.format_tags.data();
  return 0;
}

int snapref_save(void *s, const char *path, char *err, int err_len) {
  try {
    static_cast<SessionSnapshot *>(s)->save(path);
    return 0;
  } catch (const std::exception &e) {
    std::snprintf(err, (size_t)err_len, "%s", e.what());
    return -1;
  }
}

}  // extern "C"
