// Weights read from a safetensors file a tensor at a time (crates/graph/src/checkpoint.rs): the
// header parsed on opening, each tensor's bytes read from its offsets when asked for, so that a
// checkpoint of several GB is never in host memory whole.
#pragma once
#include <stdint.h>

#include <map>
#include <string>
#include <vector>

#include "tgx.h"

namespace tgx {

struct CheckpointEntry {
    tgx_dtype dtype = TGX_F32;
    size_t width = 4;  // bytes a value
    std::vector<int64_t> shape;
    uint64_t begin = 0, end = 0;  // data_offsets, from the end of the header
    size_t count() const;
};

struct Checkpoint {
    std::string path;
    int fd = -1;
    uint64_t data = 0;  // where the data after the header starts
    std::map<std::string, CheckpointEntry> entries;
    std::vector<std::string> names;  // the entries' names in order
};

tgx_status checkpoint_open(const char* path, Checkpoint** out);
void checkpoint_close(Checkpoint* ck);
// Tensor `name` as it is stored: its entry and bytes.
tgx_status checkpoint_bytes(const Checkpoint* ck, const std::string& name, const CheckpointEntry** entry,
                            std::vector<uint8_t>& bytes);
// The 2-D tensors `names` joined along their rows (checkpoint.rs:141-167), in their stored dtype
// when they share one, else in f32.
tgx_status checkpoint_rows(const Checkpoint* ck, const std::vector<std::string>& names, std::vector<uint8_t>& bytes,
                           tgx_dtype* dtype, size_t* count);

// Rows `rows` of the 2-D tensor `name` in f32, one after another (checkpoint.rs:127-139): an
// embedding lookup reading those rows alone; `columns` their width.
tgx_status checkpoint_gather(const Checkpoint* ck, const std::string& name, const int64_t* rows, int n, float* out,
                             int64_t* columns);

struct Decoder;
struct LmSide;
struct Sampler;
struct Encoder;
// A checkpoint's tensors into a model, under the names the reference's loaders read them by.
tgx_status decoder_load_checkpoint(Decoder* dec, const Checkpoint* ck, const char* prefix);
tgx_status lm_side_load_checkpoint(LmSide* s, const Checkpoint* ck);
tgx_status sampler_load_checkpoint(Sampler* s, const Checkpoint* ck);
tgx_status encoder_load_checkpoint(Encoder* e, const Checkpoint* ck);

}  // namespace tgx
