// Backend-owned storage behind a Tensor. Declarations match the reference's
// core/buffer.h:11-43 (StorageRelation, StorageIdentity, StorageAccess,
// Buffer) so backend buffers interoperate with the reference core.
#pragma once

#include <cstddef>
#include <memory>
#include <mutex>

#include "tensorcx/core/status.h"

namespace tensorcx {

enum class StorageRelation { kDisjoint, kSameRange, kPartialOverlap };

struct StorageIdentity {
  const void* token;
  std::size_t offset, bytes;
};

class StorageAccess {
 public:
  virtual ~StorageAccess() = default;
  virtual Status validate() const = 0;
  std::recursive_mutex mutex;
};

class Buffer {
 public:
  virtual ~Buffer() = default;
  virtual std::size_t nbytes() const = 0;
  virtual std::shared_ptr<StorageAccess> access() const { return {}; }
  virtual StorageIdentity storage_identity() const { return {this, 0, nbytes()}; }
  virtual StorageRelation storage_relation(const Buffer& other) const {
    if (this == &other) return StorageRelation::kSameRange;
    const StorageIdentity mine = storage_identity(), theirs = other.storage_identity();
    if (mine.token == nullptr || mine.token != theirs.token || mine.bytes == 0 || theirs.bytes == 0)
      return StorageRelation::kDisjoint;
    if (mine.offset == theirs.offset && mine.bytes == theirs.bytes) return StorageRelation::kSameRange;
    const std::size_t lo = mine.offset < theirs.offset ? mine.offset : theirs.offset;
    const std::size_t lo_bytes = mine.offset < theirs.offset ? mine.bytes : theirs.bytes;
    const std::size_t hi = mine.offset < theirs.offset ? theirs.offset : mine.offset;
    return hi - lo < lo_bytes ? StorageRelation::kPartialOverlap : StorageRelation::kDisjoint;
  }
};

}  // namespace tensorcx
