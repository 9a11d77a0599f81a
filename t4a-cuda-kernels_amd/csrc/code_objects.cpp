// The code objects that export the reference-named kernel entries, and where
// they are.
//
// The reference ships its kernels as CUDA text for the consumer to compile
// (reference src/lib.rs:32-130: `source::MODULES`, `module_of(entry)`,
// `compose`), and its design puts that compilation in a prepare step that
// runs before any numerical work and keeps loaded modules private to each
// runtime (reference docs/design/cubecl-kernel-port.md:88-109). On this target
// the compilation happens at build time: `hipcc --genco` writes one gfx950 code
// object per translation unit next to this library, so a consumer's prepare
// step is loading those files (hipModuleLoadData) and binding entries by name
// (hipModuleGetFunction). This file answers which file exports which entry and
// where the files are; it loads nothing itself.
#include <dlfcn.h>

#include <cstring>

#include "t4a/t4a.h"

namespace {

const char* const kMovementEntries[] = {
    "t4a_cuda_fill_zero",
    "t4a_cuda_fill_zero_view",
    "t4a_cuda_copy_exact",
    "t4a_cuda_materialize_strided",
    "t4a_cuda_contiguous_to_view",
    "t4a_cuda_strided_to_strided",
    "t4a_cuda_tiled_transpose",
    "t4a_cuda_broadcast_in_dim",
    "t4a_cuda_concatenate_copy",
    "t4a_cuda_fill_zero_view_any",
    "t4a_cuda_materialize_strided_any",
    "t4a_cuda_contiguous_to_view_any",
    "t4a_cuda_strided_to_strided_any",
    "t4a_cuda_broadcast_in_dim_any",
    "t4a_cuda_concatenate_copy_any",
};

const char* const kReduceEntries[] = {
    "t4a_cuda_reduce",
    "t4a_cuda_reduce_partials",
    "t4a_cuda_reduce_any",
    "t4a_cuda_reduce_partials_any",
};

struct CodeObject {
  const char* name;  // the translation unit, as the reference's module names
  const char* file;  // next to libt4a_hip.so
  const char* const* entries;
  int count;
};

const CodeObject kCodeObjects[] = {
    {"movement", "t4a_movement.gfx950.hsaco", kMovementEntries,
     static_cast<int>(sizeof(kMovementEntries) / sizeof(kMovementEntries[0]))},
    {"reduce", "t4a_reduce.gfx950.hsaco", kReduceEntries,
     static_cast<int>(sizeof(kReduceEntries) / sizeof(kReduceEntries[0]))},
};

constexpr int kCount = static_cast<int>(sizeof(kCodeObjects) / sizeof(kCodeObjects[0]));

const CodeObject* at(int index) {
  return index >= 0 && index < kCount ? &kCodeObjects[index] : nullptr;
}

}  // namespace

extern "C" {

int t4a_code_object_count(void) { return kCount; }

const char* t4a_code_object_name(int index) {
  const CodeObject* c = at(index);
  return c ? c->name : nullptr;
}

const char* t4a_code_object_file(int index) {
  const CodeObject* c = at(index);
  return c ? c->file : nullptr;
}

const char* t4a_code_object_target(void) { return "gfx950"; }

int t4a_code_object_entry_count(int index) {
  const CodeObject* c = at(index);
  return c ? c->count : 0;
}

const char* t4a_code_object_entry(int index, int entry) {
  const CodeObject* c = at(index);
  return c && entry >= 0 && entry < c->count ? c->entries[entry] : nullptr;
}

int t4a_code_object_of(const char* entry) {
  if (entry == nullptr) return -1;
  for (int i = 0; i < kCount; ++i) {
    for (int k = 0; k < kCodeObjects[i].count; ++k) {
      if (std::strcmp(kCodeObjects[i].entries[k], entry) == 0) return i;
    }
  }
  return -1;
}

int t4a_code_object_path(int index, char* path, unsigned long capacity) {
  const CodeObject* c = at(index);
  if (c == nullptr) return T4A_HIP_ERR_NOT_FOUND;
  if (path == nullptr) return T4A_HIP_ERR_NULL_ARGUMENT;
  Dl_info info;
  if (dladdr(reinterpret_cast<void*>(&t4a_code_object_path), &info) == 0 ||
      info.dli_fname == nullptr)
    return T4A_HIP_ERR_NOT_FOUND;
  const char* lib = info.dli_fname;
  const char* slash = std::strrchr(lib, '/');
  const unsigned long dir = slash ? static_cast<unsigned long>(slash - lib + 1) : 0;
  const unsigned long file = std::strlen(c->file);
  if (dir + file + 1 > capacity) return T4A_HIP_ERR_TOO_SMALL;
  std::memcpy(path, lib, dir);
  std::memcpy(path + dir, c->file, file + 1);
  return T4A_OK;
}

}  // extern "C"
