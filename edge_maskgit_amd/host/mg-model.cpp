// mg-model.cpp — GGUF v3 reader: header, metadata key/values, tensor infos, aligned data
// section; tensors are exposed as external (zero-copy) mg::Tensor objects over the mmap.
//
// File format (GGUF v3, as written by the reference's tools/convert_to_gguf.py and read by
// src/mg-model.cpp:139-201):
//   u32 magic "GGUF" | u32 version 3 | u64 n_tensors | u64 n_kv
//   n_kv x { string key | u32 value type | value }       (string = u64 length + bytes)
//   n_tensors x { string name | u32 n_dims | u64 ne[n_dims] | u32 ggml type | u64 offset }
//   data section at the next multiple of general.alignment (default 32); tensor data at
//   data_start + offset.
// Tensor types accepted: F32 (0), Q8_0 (8), Q4_K (12), I8 (24), packed int4 (100).
#include "mg-model.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <stdexcept>

namespace mg {

namespace {

enum Vt : uint32_t { U8 = 0, I8v, U16, I16, U32, I32v, F32v, BOOL, STRING, ARRAY, U64, I64, F64 };
enum Gt : uint32_t { G_F32 = 0, G_Q8_0 = 8, G_Q4_K = 12, G_I8 = 24, G_I4 = 100 };

size_t scalar_bytes(uint32_t t) {
    switch (t) {
        case U8: case I8v: case BOOL: return 1;
        case U16: case I16: return 2;
        case U32: case I32v: case F32v: return 4;
        case U64: case I64: case F64: return 8;
        default: return 0;
    }
}

struct Reader {
    const uint8_t* p;
    const uint8_t* end;
    void need(size_t n) const {
        if ((size_t)(end - p) < n) throw std::runtime_error("gguf: truncated file");
    }
    template <class T>
    T get() {
        need(sizeof(T));
        T v;
        std::memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        need(n);
        std::string s((const char*)p, (size_t)n);
        p += n;
        return s;
    }
    void skip_value(uint32_t t) {
        if (t == STRING) {
            str();
        } else if (t == ARRAY) {
            const uint32_t sub = get<uint32_t>();
            const uint64_t n = get<uint64_t>();
            for (uint64_t i = 0; i < n; i++) skip_value(sub);
        } else {
            const size_t b = scalar_bytes(t);
            if (!b) throw std::runtime_error("gguf: unknown metadata type");
            need(b);
            p += b;
        }
    }
    int64_t integer(uint32_t t) {
        switch (t) {
            case U8: case BOOL: return get<uint8_t>();
            case I8v: return get<int8_t>();
            case U16: return get<uint16_t>();
            case I16: return get<int16_t>();
            case U32: return get<uint32_t>();
            case I32v: return get<int32_t>();
            case U64: return (int64_t)get<uint64_t>();
            case I64: return get<int64_t>();
            default: throw std::runtime_error("gguf: expected an integer value");
        }
    }
};

}  // namespace

struct GgufReader {
    // one metadata entry: recognized keys go to hp, everything else is skipped
    static void kv(Reader& r, HParams& hp, uint32_t& alignment) {
        const std::string key = r.str();
        const uint32_t t = r.get<uint32_t>();
        if (t == STRING) {
            const std::string s = r.str();
            if (key == "general.architecture") hp.arch = s;
            else if (key == "general.name") hp.name = s;
            else if (key == "maskgit.quant") hp.quant = s;
            return;
        }
        if (t == F32v) {
            const float f = r.get<float>();
            if (key == "maskgit.layernorm_eps") hp.ln_eps = f;
            else if (key == "maskgit.sampling.choice_temperature") hp.choice_temperature = f;
            return;
        }
        if (t == ARRAY) {
            if (key == "maskgit.vqgan.channel_multipliers") {
                const uint32_t sub = r.get<uint32_t>();
                const uint64_t n = r.get<uint64_t>();
                hp.vq_channel_mult.clear();
                for (uint64_t i = 0; i < n; i++) hp.vq_channel_mult.push_back((int)r.integer(sub));
            } else {
                r.skip_value(t);
            }
            return;
        }
        if (t == F64) {
            r.skip_value(t);
            return;
        }
        const int64_t v = r.integer(t);
        struct { const char* k; int* dst; } ints[] = {
            {"maskgit.n_layer", &hp.n_layer}, {"maskgit.n_head", &hp.n_head},
            {"maskgit.n_embd", &hp.n_embd}, {"maskgit.n_ffn", &hp.n_ffn},
            {"maskgit.head_dim", &hp.head_dim}, {"maskgit.vocab_size", &hp.vocab_size},
            {"maskgit.n_tokens", &hp.n_tokens}, {"maskgit.n_positions", &hp.n_positions},
            {"maskgit.mask_token_id", &hp.mask_token_id}, {"maskgit.resolution", &hp.resolution},
            {"maskgit.vqgan.codebook_size", &hp.vq_codebook_size},
            {"maskgit.vqgan.embedding_dim", &hp.vq_embedding_dim},
            {"maskgit.vqgan.filters", &hp.vq_filters},
            {"maskgit.vqgan.num_res_blocks", &hp.vq_num_res_blocks},
            {"maskgit.vqgan.group_norm_groups", &hp.vq_gn_groups},
        };
        for (auto& e : ints)
            if (key == e.k) *e.dst = (int)v;
        if (key == "general.alignment" && v > 0) alignment = (uint32_t)v;
    }
};

Tensor* Model::get(const std::string& n) const {
    const auto it = tensors_.find(n);
    return it == tensors_.end() ? nullptr : it->second;
}

Tensor* Model::require(const std::string& n) const {
    Tensor* t = get(n);
    if (!t) throw std::runtime_error("gguf: missing tensor '" + n + "'");
    return t;
}

std::unique_ptr<Model> Model::load(const std::string& path, Context& ctx) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) throw std::runtime_error("gguf: cannot open " + path);
    struct stat st {};
    if (::fstat(fd, &st) != 0 || st.st_size < 24) {
        ::close(fd);
        throw std::runtime_error("gguf: cannot stat or too small: " + path);
    }
    const size_t size = (size_t)st.st_size;
    void* base = ::mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (base == MAP_FAILED) {
        ::close(fd);
        throw std::runtime_error("gguf: mmap failed: " + path);
    }
    std::unique_ptr<Model> m(new Model());
    m->base_ = base;
    m->size_ = size;
    m->fd_ = fd;                                   // released by ~Model on any throw below

    const uint8_t* b = (const uint8_t*)base;
    Reader r{b, b + size};
    if (r.get<uint32_t>() != 0x46554747u) throw std::runtime_error("gguf: bad magic in " + path);
    if (r.get<uint32_t>() != 3) throw std::runtime_error("gguf: only version 3 is supported");
    const uint64_t n_tensors = r.get<uint64_t>();
    const uint64_t n_kv = r.get<uint64_t>();
    // every tensor record takes at least 8 (name length) + 4 (rank) + 8 (one dim) + 4 (type) +
    // 8 (offset) bytes: a count the file cannot hold is rejected before anything is sized by it
    if (n_tensors > size / 32) throw std::runtime_error("gguf: tensor count larger than the file allows");
    uint32_t alignment = 32;
    for (uint64_t i = 0; i < n_kv; i++) GgufReader::kv(r, m->hp_, alignment);

    struct Info {
        std::string name;
        int n_dims;
        int64_t ne[MAX_DIMS];
        uint32_t type;
        uint64_t offset;
    };
    std::vector<Info> infos((size_t)n_tensors);
    for (Info& in : infos) {
        in.name = r.str();
        in.n_dims = (int)r.get<uint32_t>();
        if (in.n_dims < 1 || in.n_dims > MAX_DIMS) throw std::runtime_error("gguf: bad rank for " + in.name);
        for (int d = 0; d < MAX_DIMS; d++) in.ne[d] = 1;
        for (int d = 0; d < in.n_dims; d++) {
            const uint64_t v = r.get<uint64_t>();
            if (v == 0 || v > ((uint64_t)1 << 40)) throw std::runtime_error("gguf: bad dimension for " + in.name);
            in.ne[d] = (int64_t)v;
        }
        in.type = r.get<uint32_t>();
        in.offset = r.get<uint64_t>();
    }
    const size_t data0 = ((size_t)(r.p - b) + alignment - 1) / alignment * alignment;
    for (const Info& in : infos) {
        Type t;
        switch (in.type) {
            case G_F32: t = Type::F32; break;
            case G_Q8_0: t = Type::Q8_0; break;
            case G_Q4_K: t = Type::Q4_K; break;
            case G_I8: t = Type::I8; break;
            case G_I4: t = Type::I4; break;
            default: throw std::runtime_error("gguf: unsupported tensor type for " + in.name);
        }
        // bounds without overflow: the data section starts inside the file, the offset lies
        // in it, and the tensor's bytes fit after the offset; the pointer is formed only then
        double elems = 1.0;
        for (int d = 0; d < MAX_DIMS; d++) elems *= (double)in.ne[d];
        if (elems > 1e15) throw std::runtime_error("gguf: tensor too large: " + in.name);
        if (data0 > size || in.offset > size - data0) throw std::runtime_error("gguf: tensor past EOF: " + in.name);
        Tensor* x = ctx.external(t, in.n_dims, in.ne, nullptr);
        if (x->nbytes() > size - data0 - in.offset) throw std::runtime_error("gguf: tensor past EOF: " + in.name);
        x->data = const_cast<uint8_t*>(b) + data0 + in.offset;
        x->name = in.name;
        m->tensors_[in.name] = x;
    }
    return m;
}

Model::~Model() {
    if (base_) ::munmap(base_, size_);
    if (fd_ >= 0) ::close(fd_);
}

}  // namespace mg
