/*
 * adaptq/storage.h -- compressed-vector handle and storage interface.
 *
 * Same declarations as the reference's include/adaptq/storage.h:19-73
 * (StorageSlot, ADAPTQ_INVALID_SLOT, CompressResult, IStorageBackend), which
 * the kernel-backend interface (adaptq/kernel.h) takes its inputs in, so a
 * V2 runtime built against the reference's headers can use this library's
 * kernel backend.  Interface only; this library implements no storage
 * backend (its rings live in device memory behind the C ABI).
 */
#pragma once

#include <cstddef>
#include <cstdint>

namespace adaptq {

/* Index into a storage backend. */
using StorageSlot = uint32_t;
static constexpr StorageSlot ADAPTQ_INVALID_SLOT = ~StorageSlot(0);

/* One compressed K or V vector. */
struct CompressResult {
  const uint8_t *data; /* packed bytes, owned by the storage backend */
  int data_bytes;      /* length of data */
  float scale;         /* reconstruction scale (the vector's L2 norm) */
  uint8_t format_tag;  /* 0x02/0x03/0x04 packed 2/3/4-bit codes, 0xFF fp32 */
  StorageSlot slot;    /* backend slot, ADAPTQ_INVALID_SLOT if not stored */
};

struct IStorageBackend {
  virtual ~IStorageBackend() = default;
  virtual void init(int capacity, int max_slot_bytes) = 0;
  virtual void reset() = 0;
  virtual StorageSlot write(const uint8_t *data, int data_bytes, float scale,
                            uint8_t format_tag) = 0;
  virtual CompressResult read(StorageSlot slot) const = 0;
  virtual void free_slot(StorageSlot slot) = 0;
  virtual size_t bytes_used() const = 0;
  virtual size_t bytes_capacity() const = 0;
  virtual const char *name() const = 0;
};

} /* namespace adaptq */
