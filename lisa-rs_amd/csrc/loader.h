// loader.h — internal interface of the checkpoint reader (loader.cpp): the
// safetensors container (the reference's src/format/safetensor.rs) and the
// name -> slot index over several shards (src/model/weights.rs), used by the
// runner to validate and upload a checkpoint (runner.rs:337-417, 3769-3955).
#ifndef LISA_LOADER_H
#define LISA_LOADER_H

#include <cstdint>
#include <string>
#include <vector>

#include "lisa_hip.h"

// One tensor of the index: its shard, byte offset from the start of that
// shard's data region, length, dtype (LISA_DT_*) and shape (WeightSlot,
// weights.rs:7-14).
struct LisaSlotInfo {
  int shard = 0;
  uint64_t offset = 0, len = 0;
  int dtype = 0;
  std::vector<uint64_t> shape;
};

// Lookup; nullptr when absent.
const LisaSlotInfo* lisa_index_find(const LisaWeightIndex* idx, const std::string& name);
// Host address of a slot's bytes inside its shard's mapping.
const uint8_t* lisa_index_bytes(const LisaWeightIndex* idx, const LisaSlotInfo& s);
const char* lisa_dtype_name(int dtype);
// slot() of runner.rs:3930-3946: the tensor must exist with exactly this
// dtype and shape, else LISA_E_ARG with the reference's message.
int lisa_index_expect(const LisaWeightIndex* idx, const std::string& name, int dtype,
                      const std::vector<uint64_t>& shape, const LisaSlotInfo** out);
// The sorted *.safetensors files of a snapshot directory (QwenRunner::load,
// runner.rs:345-357).
int lisa_snapshot_paths(const char* dir, std::vector<std::string>* out);
int lisa_index_open_paths(const std::vector<std::string>& paths, LisaWeightIndex** out);

#endif  // LISA_LOADER_H
