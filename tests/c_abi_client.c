/* A plain C11 client of the C-ABI (include/kvx.h), built and run by
 * tests/test_c_client.py on the CPU: a host-only manager's block accessors
 * and pool table, copy specs, the block allocator and the wire framing, with
 * the reference's known answers, and the RAIDEN_SHM_* environment defaults
 * applied inside the library (a manager and a store that name no segment).
 * Exits non-zero at the first mismatch. */
#define _POSIX_C_SOURCE 200809L /* setenv, getpid, unlink */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "kvx.h"

#define EXPECT(c)                                                    \
  do {                                                               \
    if (!(c)) {                                                      \
      fprintf(stderr, "FAILED %s:%d: %s (%s)\n", __FILE__, __LINE__, #c, \
              kvx_last_error());                                     \
      return 1;                                                      \
    }                                                                \
  } while (0)

int main(void) {
  /* Host-only manager: 2 layers x 1 shard, 128-byte blocks, 4 host blocks. */
  kvx_manager_config cfg;
  memset(&cfg, 0, sizeof(cfg));
  cfg.host_alloc = KVX_HOST_MALLOC;
  cfg.num_layers = 2;
  cfg.num_shards = 1;
  cfg.slice_byte_size = 128;
  cfg.host_blocks = 4;
  kvx_manager* m = NULL;
  EXPECT(kvx_manager_create(&cfg, &m) == KVX_OK);
  EXPECT(kvx_manager_num_block_arrays(m) == 2);
  EXPECT(kvx_manager_block_bytes(m, 1) == 128);

  uint8_t payload[128];
  for (int i = 0; i < 128; ++i) payload[i] = (uint8_t)(i * 7 + 1);
  EXPECT(kvx_manager_write_block(m, 1, 2, 0, payload, sizeof(payload)) == KVX_OK);
  uint8_t back[128];
  EXPECT(kvx_manager_read_block(m, 1, 2, 0, back, sizeof(back)) == KVX_OK);
  EXPECT(memcmp(back, payload, sizeof(back)) == 0);
  EXPECT(kvx_manager_write_block(m, 1, 4, 0, payload, sizeof(payload)) == KVX_OUT_OF_RANGE);

  /* Pool table: ExplicitPoolAddressingUsesPoolBaseAndStride. */
  kvx_region_spec region = {"block", 0, 64, 64, 1, 1};
  kvx_pool_spec pool = {"kind_a", 1, 128, 64, 4, &region, 1, "dtype_a"};
  EXPECT(kvx_manager_register_pools(m, &pool, 1) == KVX_OK);
  EXPECT(kvx_manager_num_pools(m) == 1 && kvx_manager_has_explicit_pools(m) == 1);
  const uint64_t s1 = kvx_manager_host_ptr(m, 1, 0);
  EXPECT(kvx_manager_block_array_block_ptr(m, 0, 0, 2) == s1 + 128 + 2 * 64);
  int64_t ids[3] = {0, 2, 3};
  uint64_t ptrs[8];
  int64_t sizes[8], n = 0;
  EXPECT(kvx_manager_block_chunks(m, 0, 0, ids, 3, 150, ptrs, sizes, 8, &n) == KVX_OK);
  EXPECT(n == 3 && ptrs[0] == s1 + 128 && sizes[0] == 64 && ptrs[2] == s1 + 320 &&
         sizes[2] == 22);
  kvx_manager_destroy(m);

  /* Copy spec: runs of consecutive ids against compact positions. */
  int64_t run_ids[6] = {3, 4, 5, 9, 10, 2};
  int64_t src[6], dst[6], sz[6], runs = 0;
  EXPECT(kvx_offsets_impl(run_ids, 6, 1, src, dst, sz, &runs) == KVX_OK);
  EXPECT(runs == 3 && src[1] == 3 && dst[1] == 9 && sz[1] == 2);

  /* Pool geometry: ComputePoolBlockCopyExtentsTest.Basic. */
  kvx_region_spec payload_region = {"payload", 0, 1000, 1000, 1, 1};
  kvx_pool_spec p0 = {"pool0", 0, 0, 1000, 10, &payload_region, 1, ""};
  int64_t blocks[5] = {0, 1, 3, 4, 5};
  int64_t ext[8], next = 0;
  EXPECT(kvx_pool_copy_extents(&p0, blocks, 5, ext, 4, &next) == KVX_OK);
  EXPECT(next == 2 && ext[0] == 0 && ext[1] == 2000 && ext[2] == 3000 && ext[3] == 3000);

  /* Wire bytes: ChunkHeaderSerializerTest.SerializeToLittleEndian. */
  kvx_chunk_header h = {1, 0xAB, 0xCD, 0x1234, 0x5678, 24, 0x12345678u, 0x9ABCDEF0u,
                        0x11223344u, 0x0123456789ABCDEFull};
  uint8_t wire[64];
  kvx_chunk_header_serialize(&h, wire);
  const uint8_t want[8] = {0x52, 0x44, 0x01, 0x00, 0xAB, 0xCD, 0x34, 0x12};
  EXPECT(memcmp(wire, want, sizeof(want)) == 0);
  kvx_chunk_header round;
  EXPECT(kvx_chunk_header_deserialize(wire, 64, &round) == KVX_OK);
  EXPECT(round.uuid == h.uuid && round.count_or_size == h.count_or_size);
  wire[0] ^= 0xFF;
  EXPECT(kvx_chunk_header_deserialize(wire, 64, &round) == KVX_INVALID_ARGUMENT);

  /* Block allocator: ascending free ids, locked. */
  kvx_block_manager* b = NULL;
  EXPECT(kvx_block_manager_create(8, &b) == KVX_OK);
  int32_t got[3];
  EXPECT(kvx_block_manager_allocate(b, 3, 1, got) == KVX_OK);
  EXPECT(got[0] == 0 && got[1] == 1 && got[2] == 2);
  kvx_block_manager_destroy(b);

  /* RAIDEN_SHM_*: a manager asking for the reference's default allocator
   * (KVX_HOST_AUTO) and naming no segment gets the shm tier under
   * RAIDEN_SHM_KEY, warm on its second creation; a store naming no metadata
   * table gets "<key>_metadata". */
  char key[64], path[96], meta[96];
  snprintf(key, sizeof(key), "kvx_c_env_%d", (int)getpid());
  snprintf(path, sizeof(path), "/dev/shm/%s", key);
  snprintf(meta, sizeof(meta), "/dev/shm/%s_metadata", key);
  EXPECT(setenv("RAIDEN_SHM_KEY", key, 1) == 0);
  EXPECT(setenv("RAIDEN_SHM_MODEL_UID", "c_client_model", 1) == 0);
  kvx_manager_config ec;
  memset(&ec, 0, sizeof(ec));
  ec.host_alloc = KVX_HOST_AUTO;
  ec.num_layers = 2;
  ec.num_shards = 1;
  ec.slice_byte_size = 128;
  ec.host_blocks = 4;
  kvx_manager* e1 = NULL;
  EXPECT(kvx_manager_create(&ec, &e1) == KVX_OK);
  EXPECT(kvx_manager_host_alloc(e1) == KVX_HOST_SHM);
  EXPECT(kvx_manager_shm_warm(e1) == 0);
  EXPECT(access(path, F_OK) == 0);
  EXPECT(kvx_manager_write_block(e1, 1, 3, 0, payload, sizeof(payload)) == KVX_OK);
  kvx_manager_destroy(e1);
  kvx_manager* e2 = NULL;
  EXPECT(kvx_manager_create(&ec, &e2) == KVX_OK);
  EXPECT(kvx_manager_shm_warm(e2) == 1);
  EXPECT(kvx_manager_read_block(e2, 1, 3, 0, back, sizeof(back)) == KVX_OK);
  EXPECT(memcmp(back, payload, sizeof(back)) == 0);
  kvx_manager_destroy(e2);
  /* Another schema uid: the segment is reformatted (cold). */
  EXPECT(setenv("RAIDEN_SHM_MODEL_UID", "other_model", 1) == 0);
  kvx_manager* e3 = NULL;
  EXPECT(kvx_manager_create(&ec, &e3) == KVX_OK);
  EXPECT(kvx_manager_shm_warm(e3) == 0);
  kvx_manager_destroy(e3);

  kvx_store_config sc;
  memset(&sc, 0, sizeof(sc));
  sc.capacity = 4;
  sc.job_name = "job";
  sc.job_replica_id = "0";
  sc.data_name = "cache";
  sc.num_shards = 1;
  sc.store_server_ip = "127.0.0.1";
  kvx_store* st = NULL;
  EXPECT(kvx_store_create(&sc, &st) == KVX_OK);
  EXPECT(access(meta, F_OK) == 0);
  kvx_store_destroy(st);
  unlink(path);
  unlink(meta);
  EXPECT(unsetenv("RAIDEN_SHM_KEY") == 0);
  /* shm without a key anywhere is refused. */
  ec.host_alloc = KVX_HOST_SHM;
  EXPECT(kvx_manager_create(&ec, &e1) == KVX_INVALID_ARGUMENT);
  puts("c client ok");
  return 0;
}
