// The safetensors reader (crates/graph/src/checkpoint.rs) and the loaders that write a checkpoint's
// tensors into a decoder, an LM side, a sampler or an encoder under the names the model's
// loaders give them (decode.rs:738-776 load_stack, lm_side.rs:496-533 load_lm_side,
// local/dit.rs:329-365 load_sampler, local/encoder.rs:129-162 load_encoder). A file holds an
// 8-byte little-endian header length, the header (a JSON object: for each tensor its dtype, shape
// and data_offsets; "__metadata__" aside), then the tensors' bytes.
#include "checkpoint.hpp"

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>

#include "handles.hpp"

namespace tgx {

namespace {

// ---- the header's JSON: objects, arrays, strings, numbers and the three literals ----

struct Json {
    enum Kind { NUL, BOOL, NUMBER, STRING, ARRAY, OBJECT } kind = NUL;
    double number = 0;
    bool integral = false;
    int64_t integer = 0;
    std::string text;
    std::vector<Json> items;
    std::vector<std::pair<std::string, Json>> fields;

    const Json* field(const char* name) const {
        for (const auto& f : fields)
            if (f.first == name) return &f.second;
        return nullptr;
    }
};

struct JsonParser {
    const char* p;
    const char* end;
    std::string error;
    int depth = 0;

    void space() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
    }
    bool fail_at(const char* why) {
        if (error.empty()) error = why;
        return false;
    }
    bool literal(const char* word) {
        const size_t n = std::strlen(word);
        if ((size_t)(end - p) < n || std::memcmp(p, word, n) != 0) return fail_at("a bad literal");
        p += n;
        return true;
    }
    bool string(std::string& out) {
        if (p >= end || *p != '"') return fail_at("a string expected");
        ++p;
        while (p < end && *p != '"') {
            char c = *p++;
            if (c != '\\') {
                out.push_back(c);
                continue;
            }
            if (p >= end) return fail_at("an escape cut off");
            c = *p++;
            switch (c) {
                case '"': out.push_back('"'); break;
                case '\\': out.push_back('\\'); break;
                case '/': out.push_back('/'); break;
                case 'b': out.push_back('\b'); break;
                case 'f': out.push_back('\f'); break;
                case 'n': out.push_back('\n'); break;
                case 'r': out.push_back('\r'); break;
                case 't': out.push_back('\t'); break;
                case 'u': {
                    if (end - p < 4) return fail_at("a \\u escape cut off");
                    unsigned v = 0;
                    for (int i = 0; i < 4; ++i) {
                        const char h = *p++;
                        v <<= 4;
                        if (h >= '0' && h <= '9') v |= h - '0';
                        else if (h >= 'a' && h <= 'f') v |= h - 'a' + 10;
                        else if (h >= 'A' && h <= 'F') v |= h - 'A' + 10;
                        else return fail_at("a bad \\u escape");
                    }
                    // UTF-8 of the code unit (names are ASCII in practice; surrogates kept as they are)
                    if (v < 0x80) {
                        out.push_back((char)v);
                    } else if (v < 0x800) {
                        out.push_back((char)(0xC0 | (v >> 6)));
                        out.push_back((char)(0x80 | (v & 0x3F)));
                    } else {
                        out.push_back((char)(0xE0 | (v >> 12)));
                        out.push_back((char)(0x80 | ((v >> 6) & 0x3F)));
                        out.push_back((char)(0x80 | (v & 0x3F)));
                    }
                    break;
                }
                default: return fail_at("a bad escape");
            }
        }
        if (p >= end) return fail_at("a string cut off");
        ++p;
        return true;
    }
    bool number(Json& out) {
        const char* start = p;
        bool integral = true;
        if (p < end && *p == '-') ++p;
        while (p < end && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '+' || *p == '-')) {
            if (*p == '.' || *p == 'e' || *p == 'E') integral = false;
            ++p;
        }
        if (p == start) return fail_at("a value expected");
        const std::string s(start, p);
        char* stop = nullptr;
        out.kind = Json::NUMBER;
        out.number = std::strtod(s.c_str(), &stop);
        if (!stop || *stop) return fail_at("a bad number");
        out.integral = integral;
        if (integral) {
            errno = 0;
            out.integer = std::strtoll(s.c_str(), &stop, 10);
            if (errno || *stop) return fail_at("an integer out of range");
        }
        return true;
    }
    bool value(Json& out) {
        if (++depth > 64) return fail_at("nested too deep");
        space();
        if (p >= end) return fail_at("a value expected");
        bool ok = true;
        if (*p == '{') {
            ++p;
            out.kind = Json::OBJECT;
            space();
            if (p < end && *p == '}') {
                ++p;
            } else {
                for (;;) {
                    space();
                    std::string key;
                    if (!string(key)) return false;
                    space();
                    if (p >= end || *p != ':') return fail_at("':' expected");
                    ++p;
                    Json v;
                    if (!value(v)) return false;
                    out.fields.emplace_back(std::move(key), std::move(v));
                    space();
                    if (p < end && *p == ',') {
                        ++p;
                        continue;
                    }
                    if (p < end && *p == '}') {
                        ++p;
                        break;
                    }
                    return fail_at("',' or '}' expected");
                }
            }
        } else if (*p == '[') {
            ++p;
            out.kind = Json::ARRAY;
            space();
            if (p < end && *p == ']') {
                ++p;
            } else {
                for (;;) {
                    Json v;
                    if (!value(v)) return false;
                    out.items.push_back(std::move(v));
                    space();
                    if (p < end && *p == ',') {
                        ++p;
                        continue;
                    }
                    if (p < end && *p == ']') {
                        ++p;
                        break;
                    }
                    return fail_at("',' or ']' expected");
                }
            }
        } else if (*p == '"') {
            out.kind = Json::STRING;
            ok = string(out.text);
        } else if (*p == 't') {
            out.kind = Json::BOOL;
            out.number = 1;
            ok = literal("true");
        } else if (*p == 'f') {
            out.kind = Json::BOOL;
            ok = literal("false");
        } else if (*p == 'n') {
            ok = literal("null");
        } else {
            ok = number(out);
        }
        --depth;
        return ok;
    }
};

tgx_status bad(const std::string& path, const std::string& why) { return fail(TGX_E_WEIGHTS, path + ": " + why); }

bool read_at(int fd, void* dst, size_t bytes, uint64_t offset) {
    uint8_t* d = static_cast<uint8_t*>(dst);
    while (bytes) {
        const ssize_t got = pread(fd, d, bytes, (off_t)offset);
        if (got <= 0) return false;
        d += got;
        bytes -= (size_t)got;
        offset += (uint64_t)got;
    }
    return true;
}

}  // namespace

size_t CheckpointEntry::count() const {
    size_t n = 1;
    for (int64_t d : shape) n *= (size_t)d;
    return n;
}

// Checkpoint::open (checkpoint.rs:36-71): the header's length (at most 100 MiB), the header, and
// every entry's dtype (BF16, F16 or F32), shape and offsets, checked against each other and the
// file's length.
tgx_status checkpoint_open(const char* path, Checkpoint** out) {
    if (!path || !out) return fail(TGX_E_ARG, "null path or output");
    *out = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return bad(path, std::strerror(errno));
    auto fail_closed = [&](const std::string& why) {
        close(fd);
        return bad(path, why);
    };
    struct stat st {};
    if (fstat(fd, &st) != 0) return fail_closed(std::strerror(errno));
    uint8_t len_bytes[8];
    if (!read_at(fd, len_bytes, 8, 0)) return fail_closed("shorter than a header length");
    uint64_t len = 0;
    for (int i = 7; i >= 0; --i) len = (len << 8) | len_bytes[i];
    if (len > (100ull << 20)) return fail_closed("a header of " + std::to_string(len) + " bytes");
    if (8 + len > (uint64_t)st.st_size) return fail_closed("a header past the end of the file");
    std::string header(len, '\0');
    if (!read_at(fd, header.data(), len, 8)) return fail_closed("the header cut off");
    JsonParser parser{header.data(), header.data() + header.size()};
    Json root;
    if (!parser.value(root)) return fail_closed("the header: " + parser.error);
    parser.space();
    if (parser.p != parser.end) return fail_closed("the header: text after the object");
    if (root.kind != Json::OBJECT) return fail_closed("the header is not an object");
    Checkpoint* ck = new Checkpoint();
    ck->path = path;
    ck->fd = fd;
    ck->data = 8 + len;
    const uint64_t data_bytes = (uint64_t)st.st_size - ck->data;
    for (const auto& [name, v] : root.fields) {
        if (name == "__metadata__") continue;
        auto refuse = [&](const std::string& why) {
            checkpoint_close(ck);
            return bad(path, name + ": " + why);
        };
        const Json* dtype = v.field("dtype");
        const Json* shape = v.field("shape");
        const Json* offsets = v.field("data_offsets");
        if (v.kind != Json::OBJECT || !dtype || !shape || !offsets || dtype->kind != Json::STRING || shape->kind != Json::ARRAY ||
            offsets->kind != Json::ARRAY || offsets->items.size() != 2)
            return refuse("not a tensor entry");
        CheckpointEntry e;
        if (dtype->text == "BF16") {
            e.dtype = TGX_BF16;
            e.width = 2;
        } else if (dtype->text == "F16") {
            e.dtype = TGX_F16;
            e.width = 2;
        } else if (dtype->text == "F32") {
            e.dtype = TGX_F32;
            e.width = 4;
        } else {
            return refuse(dtype->text + " weights");
        }
        for (const Json& d : shape->items) {
            if (d.kind != Json::NUMBER || !d.integral || d.integer < 0) return refuse("a bad shape");
            e.shape.push_back(d.integer);
        }
        for (int i = 0; i < 2; ++i)
            if (offsets->items[i].kind != Json::NUMBER || !offsets->items[i].integral || offsets->items[i].integer < 0)
                return refuse("bad data_offsets");
        e.begin = (uint64_t)offsets->items[0].integer;
        e.end = (uint64_t)offsets->items[1].integer;
        if (e.end < e.begin || e.end > data_bytes) return refuse("data_offsets past the end of the file");
        // checkpoint.rs:83-99: the bytes must be the shape's
        if (e.end - e.begin != (uint64_t)(e.count() * e.width))
            return refuse(std::to_string(e.end - e.begin) + " bytes for " + std::to_string(e.count()) + " " + dtype->text);
        ck->entries.emplace(name, std::move(e));
    }
    for (const auto& kv : ck->entries) ck->names.push_back(kv.first);
    *out = ck;
    return TGX_OK;
}

void checkpoint_close(Checkpoint* ck) {
    if (!ck) return;
    if (ck->fd >= 0) close(ck->fd);
    delete ck;
}

tgx_status checkpoint_bytes(const Checkpoint* ck, const std::string& name, const CheckpointEntry** entry,
                            std::vector<uint8_t>& bytes) {
    auto it = ck->entries.find(name);
    if (it == ck->entries.end()) return bad(ck->path, name + ": no such tensor");
    const CheckpointEntry& e = it->second;
    bytes.resize(e.end - e.begin);
    if (!read_at(ck->fd, bytes.data(), bytes.size(), ck->data + e.begin)) return bad(ck->path, name + ": a short read");
    if (entry) *entry = &e;
    return TGX_OK;
}

tgx_status checkpoint_rows(const Checkpoint* ck, const std::vector<std::string>& names, std::vector<uint8_t>& bytes,
                           tgx_dtype* dtype, size_t* count) {
    std::vector<std::vector<uint8_t>> parts(names.size());
    std::vector<const CheckpointEntry*> entries(names.size());
    int64_t columns = -1;
    bool same = true;
    for (size_t i = 0; i < names.size(); ++i) {
        TGX_TRY(checkpoint_bytes(ck, names[i], &entries[i], parts[i]));
        const CheckpointEntry& e = *entries[i];
        if (e.shape.size() != 2) return bad(ck->path, names[i] + ": not 2-D");
        if (columns < 0) columns = e.shape[1];
        if (e.shape[1] != columns)
            return bad(ck->path, names[i] + ": " + std::to_string(e.shape[1]) + " columns, not " + std::to_string(columns));
        same = same && e.dtype == entries[0]->dtype;
    }
    size_t total = 0;
    for (const CheckpointEntry* e : entries) total += e->count();
    bytes.clear();
    if (same) {
        *dtype = entries.empty() ? TGX_F32 : entries[0]->dtype;
        for (const auto& part : parts) bytes.insert(bytes.end(), part.begin(), part.end());
    } else {
        *dtype = TGX_F32;
        for (size_t i = 0; i < parts.size(); ++i) {
            const std::vector<float> v = as_f32(parts[i].data(), entries[i]->dtype, entries[i]->count());
            const uint8_t* b = reinterpret_cast<const uint8_t*>(v.data());
            bytes.insert(bytes.end(), b, b + v.size() * 4);
        }
    }
    *count = total;
    return TGX_OK;
}

tgx_status checkpoint_gather(const Checkpoint* ck, const std::string& name, const int64_t* rows, int n, float* out,
                             int64_t* columns_out) {
    auto it = ck->entries.find(name);
    if (it == ck->entries.end()) return bad(ck->path, name + ": no such tensor");
    const CheckpointEntry& e = it->second;
    if (e.shape.size() != 2) return bad(ck->path, name + ": not 2-D");
    const int64_t count = e.shape[0], columns = e.shape[1];
    *columns_out = columns;
    std::vector<uint8_t> bytes((size_t)columns * e.width);
    for (int i = 0; i < n; ++i) {
        if (rows[i] < 0 || rows[i] >= count) return bad(ck->path, name + ": row " + std::to_string(rows[i]) + " of " + std::to_string(count));
        if (!read_at(ck->fd, bytes.data(), bytes.size(), ck->data + e.begin + (uint64_t)rows[i] * bytes.size()))
            return bad(ck->path, name + ": a short read");
        const std::vector<float> v = as_f32(bytes.data(), e.dtype, (size_t)columns);
        std::memcpy(out + (size_t)i * columns, v.data(), v.size() * 4);
    }
    return TGX_OK;
}

namespace {

using Loader = tgx_status (*)(void* target, const char* name, const void* data, tgx_dtype dtype, size_t count);

// One tensor of the checkpoint under `want`, joined from `names` when there are several.
tgx_status load_one(const Checkpoint* ck, void* target, Loader load, const std::string& want, const std::vector<std::string>& names) {
    std::vector<uint8_t> bytes;
    tgx_dtype dtype = TGX_F32;
    size_t count = 0;
    if (names.size() == 1) {
        const CheckpointEntry* e = nullptr;
        TGX_TRY(checkpoint_bytes(ck, names[0], &e, bytes));
        dtype = e->dtype;
        count = e->count();
    } else {
        TGX_TRY(checkpoint_rows(ck, names, bytes, &dtype, &count));
    }
    return load(target, want.c_str(), bytes.data(), dtype, count);
}

// load_stack (decode.rs:738-776) and local::Stack::load (local/mod.rs:658-700): each layer's
// q/k/v and gate/up joined along their rows, then the final norm, from `prefix` in the
// checkpoint to `to` in the target's names.
tgx_status load_stack_from(const Checkpoint* ck, void* target, Loader load, int layers, const std::string& prefix,
                           const std::string& to) {
    for (int l = 0; l < layers; ++l) {
        const std::string at = prefix + "layers." + std::to_string(l) + ".";
        const std::string mine = to + "layers." + std::to_string(l) + ".";
        TGX_TRY(load_one(ck, target, load, mine + "qkv_proj",
                         {at + "self_attn.q_proj.weight", at + "self_attn.k_proj.weight", at + "self_attn.v_proj.weight"}));
        TGX_TRY(load_one(ck, target, load, mine + "o_proj", {at + "self_attn.o_proj.weight"}));
        TGX_TRY(load_one(ck, target, load, mine + "gate_up_proj", {at + "mlp.gate_proj.weight", at + "mlp.up_proj.weight"}));
        TGX_TRY(load_one(ck, target, load, mine + "down_proj", {at + "mlp.down_proj.weight"}));
        TGX_TRY(load_one(ck, target, load, mine + "input_layernorm", {at + "input_layernorm.weight"}));
        TGX_TRY(load_one(ck, target, load, mine + "post_attention_layernorm", {at + "post_attention_layernorm.weight"}));
    }
    return load_one(ck, target, load, to + "norm", {prefix + "norm.weight"});
}

tgx_status as_decoder(void* t, const char* n, const void* d, tgx_dtype dt, size_t c) {
    return decoder_load(static_cast<Decoder*>(t), n, d, dt, c);
}
tgx_status as_lm_side(void* t, const char* n, const void* d, tgx_dtype dt, size_t c) {
    return lm_side_load(static_cast<LmSide*>(t), n, d, dt, c);
}
tgx_status as_sampler(void* t, const char* n, const void* d, tgx_dtype dt, size_t c) {
    return sampler_load(static_cast<Sampler*>(t), n, d, dt, c);
}
tgx_status as_encoder(void* t, const char* n, const void* d, tgx_dtype dt, size_t c) {
    return encoder_load(static_cast<Encoder*>(t), n, d, dt, c);
}

}  // namespace

tgx_status decoder_load_checkpoint(Decoder* dec, const Checkpoint* ck, const char* prefix) {
    return load_stack_from(ck, dec, as_decoder, dec->shape.layers, prefix ? prefix : "", "");
}

// load_lm_side (lm_side.rs:496-533): both stacks, then each head's weight and bias.
tgx_status lm_side_load_checkpoint(LmSide* s, const Checkpoint* ck) {
    TGX_TRY(load_stack_from(ck, s, as_lm_side, s->base->shape.layers, "base_lm.", "base_lm."));
    TGX_TRY(load_stack_from(ck, s, as_lm_side, s->residual->shape.layers, "residual_lm.", "residual_lm."));
    for (const LmHead& h : lm_side_heads()) {
        TGX_TRY(load_one(ck, s, as_lm_side, std::string(h.name) + ".weight", {std::string(h.name) + ".weight"}));
        if (h.bias) TGX_TRY(load_one(ck, s, as_lm_side, std::string(h.name) + ".bias", {std::string(h.name) + ".bias"}));
    }
    return TGX_OK;
}

// load_sampler (local/dit.rs:329-365): the DiT's stack under feat_decoder.estimator.decoder., its
// in/cond/out projections and the two time MLPs (TimeMlp::read, dit.rs:387-407).
tgx_status sampler_load_checkpoint(Sampler* s, const Checkpoint* ck) {
    const std::string prefix = "feat_decoder.estimator.";
    TGX_TRY(load_stack_from(ck, s, as_sampler, s->shape.layers, prefix + "decoder.", ""));
    for (const char* p : {"in_proj", "cond_proj", "out_proj"})
        for (const char* part : {".weight", ".bias"}) {
            const std::string n = std::string(p) + part;
            TGX_TRY(load_one(ck, s, as_sampler, n, {prefix + n}));
        }
    for (const char* m : {"time_mlp", "delta_time_mlp"})
        for (const char* layer : {".linear_1", ".linear_2"})
            for (const char* part : {".weight", ".bias"}) {
                const std::string n = std::string(m) + layer + part;
                TGX_TRY(load_one(ck, s, as_sampler, n, {prefix + n}));
            }
    return TGX_OK;
}

// load_encoder (local/encoder.rs:129-162): the stack under feat_encoder.encoder., the learned token
// and in_proj.
tgx_status encoder_load_checkpoint(Encoder* e, const Checkpoint* ck) {
    const std::string prefix = "feat_encoder.";
    TGX_TRY(load_stack_from(ck, e, as_encoder, e->shape.layers, prefix + "encoder.", ""));
    for (const char* n : {"special_token", "in_proj.weight", "in_proj.bias"}) TGX_TRY(load_one(ck, e, as_encoder, n, {prefix + n}));
    return TGX_OK;
}

}  // namespace tgx

using namespace tgx;

extern "C" {

tgx_status tgx_checkpoint_open(const char* path, tgx_checkpoint** out) {
    clear_error();
    if (!out) return fail(TGX_E_ARG, "null output");
    *out = nullptr;
    Checkpoint* ck = nullptr;
    TGX_TRY(checkpoint_open(path, &ck));
    *out = new tgx_checkpoint{ck};
    return TGX_OK;
}

void tgx_checkpoint_close(tgx_checkpoint* ck) {
    if (!ck) return;
    checkpoint_close(ck->ck);
    delete ck;
}

tgx_status tgx_checkpoint_count(const tgx_checkpoint* ck, int* out) {
    clear_error();
    if (!ck || !out) return fail(TGX_E_ARG, "null checkpoint or output");
    *out = (int)ck->ck->names.size();
    return TGX_OK;
}

tgx_status tgx_checkpoint_name(const tgx_checkpoint* ck, int index, char* out, size_t capacity) {
    clear_error();
    if (!ck || !out || !capacity) return fail(TGX_E_ARG, "null checkpoint or output");
    if (index < 0 || (size_t)index >= ck->ck->names.size()) return fail(TGX_E_ARG, "tensor " + std::to_string(index) + " of " + std::to_string(ck->ck->names.size()));
    const std::string& n = ck->ck->names[index];
    if (n.size() + 1 > capacity) return fail(TGX_E_ARG, "a name of " + std::to_string(n.size()) + " bytes");
    std::memcpy(out, n.c_str(), n.size() + 1);
    return TGX_OK;
}

tgx_status tgx_checkpoint_shape(const tgx_checkpoint* ck, const char* name, int64_t* dims, int max, int* ndims, tgx_dtype* dtype) {
    clear_error();
    if (!ck || !name || !ndims) return fail(TGX_E_ARG, "null checkpoint, name or output");
    auto it = ck->ck->entries.find(name);
    if (it == ck->ck->entries.end()) return bad(ck->ck->path, std::string(name) + ": no such tensor");
    const CheckpointEntry& e = it->second;
    *ndims = (int)e.shape.size();
    if (dtype) *dtype = e.dtype;
    for (int i = 0; i < *ndims && i < max && dims; ++i) dims[i] = e.shape[i];
    return TGX_OK;
}

tgx_status tgx_checkpoint_read(const tgx_checkpoint* ck, const char* name, float* out, size_t count) {
    clear_error();
    if (!ck || !name || !out) return fail(TGX_E_ARG, "null checkpoint, name or output");
    std::vector<uint8_t> bytes;
    const CheckpointEntry* e = nullptr;
    TGX_TRY(checkpoint_bytes(ck->ck, name, &e, bytes));
    if (count != e->count()) return bad(ck->ck->path, std::string(name) + ": " + std::to_string(e->count()) + " values, not " + std::to_string(count));
    const std::vector<float> v = as_f32(bytes.data(), e->dtype, e->count());
    std::memcpy(out, v.data(), v.size() * 4);
    return TGX_OK;
}

tgx_status tgx_checkpoint_gather(const tgx_checkpoint* ck, const char* name, const int64_t* rows, int n, float* out) {
    clear_error();
    if (!ck || !name || (n > 0 && (!rows || !out))) return fail(TGX_E_ARG, "null checkpoint, name, rows or output");
    int64_t columns = 0;
    return checkpoint_gather(ck->ck, name, rows, n, out, &columns);
}

tgx_status tgx_decoder_load_checkpoint(tgx_decoder* dec, const tgx_checkpoint* ck, const char* prefix) {
    clear_error();
    if (!dec || !ck) return fail(TGX_E_ARG, "null decoder or checkpoint");
    return decoder_load_checkpoint(dec->dec, ck->ck, prefix);
}

tgx_status tgx_lm_side_load_checkpoint(tgx_lm_side* s, const tgx_checkpoint* ck) {
    clear_error();
    if (!s || !ck) return fail(TGX_E_ARG, "null LM side or checkpoint");
    return lm_side_load_checkpoint(s->s, ck->ck);
}

tgx_status tgx_sampler_load_checkpoint(tgx_sampler* s, const tgx_checkpoint* ck) {
    clear_error();
    if (!s || !ck) return fail(TGX_E_ARG, "null sampler or checkpoint");
    return sampler_load_checkpoint(s->s, ck->ck);
}

tgx_status tgx_encoder_load_checkpoint(tgx_encoder* e, const tgx_checkpoint* ck) {
    clear_error();
    if (!e || !ck) return fail(TGX_E_ARG, "null encoder or checkpoint");
    return encoder_load_checkpoint(e->e, ck->ck);
}

}  // extern "C"
