// The RAIDEN_SHM_* environment defaults of the reference's host tier, read in
// the library so every caller of the C-ABI inherits them:
//   RAIDEN_SHM_KEY          selects the shared-memory host allocator and names
//                           its segment (tpu_sync/core/utils.h:48-91);
//   RAIDEN_SHM_MODEL_UID    the segment's schema model uid, else
//                           "default_model" (utils.h:54-61,
//                           tpu_sync/kv_cache/kv_cache_store_wrapper.cc:120-123;
//                           an empty value counts as unset here, since an empty
//                           uid in the schema means "default_model" throughout
//                           this library);
//   RAIDEN_SHM_SERVER_NAME  when non-empty, "_<name>" after the segment key
//                           (tpu_sync/core/host_memory_allocator.cc:267-271) and
//                           after the metadata table key
//                           (kv_cache_store_wrapper.cc:46-58).
#ifndef KVX_HOST_RAIDEN_ENV_H_
#define KVX_HOST_RAIDEN_ENV_H_

#include <cstdlib>
#include <string>

namespace kvx {

inline std::string ShmKeyFromEnv() {
  const char* v = std::getenv("RAIDEN_SHM_KEY");
  return v != nullptr ? v : "";
}

inline std::string ShmModelUidFromEnv() {
  const char* v = std::getenv("RAIDEN_SHM_MODEL_UID");
  return v != nullptr && v[0] != '\0' ? v : "default_model";
}

inline std::string ShmServerNameFromEnv() {
  const char* v = std::getenv("RAIDEN_SHM_SERVER_NAME");
  return v != nullptr ? v : "";
}

// "<RAIDEN_SHM_KEY>_metadata[_<RAIDEN_SHM_SERVER_NAME>]", or "" (no table)
// when RAIDEN_SHM_KEY is unset or empty.
inline std::string MetadataShmKeyFromEnv() {
  std::string key = ShmKeyFromEnv();
  if (key.empty()) return "";
  key += "_metadata";
  const std::string server = ShmServerNameFromEnv();
  if (!server.empty()) key += "_" + server;
  return key;
}

}  // namespace kvx

#endif  // KVX_HOST_RAIDEN_ENV_H_
