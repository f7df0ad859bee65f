// .rinn reader.  File layout (loader.cpp:19-26,90-103 and the writer,
// tools/convert_llama_to_rinn.py:97-123), little-endian:
//   [0, 512)        header: "RINN", u32 version @4, u32 tensor count @8,
//                   u64 config offset @16, u64 config bytes @24,
//                   u64 index offset @32, u64 index bytes @40,
//                   u64 data offset @48
//   config          JSON object (the ModelConfig keys, "block_size" for
//                   max_seq_len, "layers": [{"type": ..}, ..])
//   index           per tensor: u16 name length, name bytes, 4 x i32 shape
//                   (trailing zeros past the rank), u8 quant type,
//                   u16 block size, u64 absolute offset, u64 byte size
//   data            tensor bytes at their offsets
#include "core/loader.h"
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <sys/stat.h>
#include <vector>

namespace {

struct File {
    FILE* f = nullptr;
    ~File() { if (f) fclose(f); }
    bool read_at(uint64_t off, void* dst, size_t n) {
        if (fseeko(f, (off_t)off, SEEK_SET) != 0) return false;
        return fread(dst, 1, n, f) == n;
    }
};

uint64_t le64(const uint8_t* p) {
    uint64_t v = 0;
    for (int i = 7; i >= 0; i--) v = (v << 8) | p[i];
    return v;
}
uint32_t le32(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }
uint16_t le16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

struct Spec {
    std::string name;
    int shape[4];
    int n_dim;
    int quant_type;
    uint64_t offset, size;
};

bool fail(std::string* err, const std::string& m) {
    if (err) *err = m;
    return false;
}

}  // namespace

bool load_rinn(const std::string& path_in, ModelConfig& cfg, TensorMap& tensors, std::string* err) {
    std::string path = path_in;
    struct stat st{};
    if (stat(path.c_str(), &st) == 0 && S_ISDIR(st.st_mode)) path += "/weights.rinn";
    File fh;
    fh.f = fopen(path.c_str(), "rb");
    if (!fh.f) return fail(err, "rinn: cannot open " + path);
    uint8_t hdr[512];
    if (fread(hdr, 1, sizeof hdr, fh.f) != sizeof hdr) return fail(err, "rinn: short header in " + path);
    if (memcmp(hdr, "RINN", 4) != 0) return fail(err, "rinn: bad magic in " + path);
    const uint32_t n_tensors = le32(hdr + 8);
    const uint64_t cfg_off = le64(hdr + 16), cfg_sz = le64(hdr + 24);
    const uint64_t idx_off = le64(hdr + 32), idx_sz = le64(hdr + 40);
    if (fseeko(fh.f, 0, SEEK_END) != 0) return fail(err, "rinn: seek failed");
    const uint64_t file_sz = (uint64_t)ftello(fh.f);
    if (cfg_off > file_sz || cfg_sz > file_sz - cfg_off || idx_off > file_sz || idx_sz > file_sz - idx_off)
        return fail(err, "rinn: config or index past the end of " + path);

    std::string json(cfg_sz, '\0');
    if (!fh.read_at(cfg_off, &json[0], cfg_sz)) return fail(err, "rinn: cannot read the config");
    ModelConfig c;
    std::string perr;
    if (!parse_config(json, c, &perr)) return fail(err, "rinn: " + perr);

    std::vector<uint8_t> idx(idx_sz);
    if (!fh.read_at(idx_off, idx.data(), idx_sz)) return fail(err, "rinn: cannot read the index");
    std::vector<Spec> specs;
    size_t p = 0;
    while (p < idx_sz) {
        if (idx_sz - p < 2) return fail(err, "rinn: truncated index");
        const size_t nl = le16(&idx[p]);
        p += 2;
        if (idx_sz - p < nl + 16 + 1 + 2 + 16) return fail(err, "rinn: truncated index");
        Spec s;
        s.name.assign((const char*)&idx[p], nl);
        p += nl;
        for (int i = 0; i < 4; i++, p += 4) s.shape[i] = (int)le32(&idx[p]);
        s.quant_type = idx[p];
        p += 1 + 2;                                   // quant type, block size
        s.offset = le64(&idx[p]);
        s.size = le64(&idx[p + 8]);
        p += 16;
        int nd = 4;
        while (nd > 0 && s.shape[nd - 1] == 0) nd--;
        s.n_dim = nd;
        specs.push_back(std::move(s));
    }
    if (specs.size() != n_tensors) return fail(err, "rinn: index holds a different tensor count than the header");

    TensorMap loaded;
    auto abort_load = [&](const std::string& m) {
        loaded.free_all();
        return fail(err, m);
    };
    std::vector<uint8_t> buf;
    for (const Spec& s : specs) {
        WeightTensor t;
        t.quant_type = (QuantType)s.quant_type;
        t.n_dim = s.n_dim;
        t.n_elems = 1;
        // every dim inside the rank positive, the element count far from
        // int64 overflow (byte sizes are derived from it)
        for (int i = 0; i < s.n_dim; i++) {
            if (s.shape[i] <= 0 || __builtin_mul_overflow(t.n_elems, (int64_t)s.shape[i], &t.n_elems) ||
                t.n_elems > ((int64_t)1 << 48))
                return abort_load("rinn: tensor " + s.name + " has a non-positive or oversized shape");
            t.shape[i] = s.shape[i];
        }
        size_t bytes;
        if (t.quant_type == QuantType::FP32) bytes = (size_t)t.n_elems * sizeof(float);
        else if (t.quant_type == QuantType::Q4_0 || t.quant_type == QuantType::Q4_0F)
            bytes = quantized_size(t.n_elems, t.quant_type);
        else
            return abort_load("rinn: unsupported quant_type " + std::to_string(s.quant_type) + " for " + s.name);
        if (s.n_dim == 0 || bytes > s.size || s.offset > file_sz || bytes > file_sz - s.offset)
            return abort_load("rinn: tensor " + s.name + " past the end of the file or smaller than its shape");
        buf.resize(bytes);
        if (!fh.read_at(s.offset, buf.data(), bytes)) return abort_load("rinn: cannot read " + s.name);
        if (hipMalloc(&t.data, bytes) != hipSuccess) return abort_load("rinn: device allocation failed for " + s.name);
        t.owned = true;
        if (hipMemcpy(t.data, buf.data(), bytes, hipMemcpyHostToDevice) != hipSuccess) {
            t.free();
            return abort_load("rinn: upload failed for " + s.name);
        }
        loaded.add(s.name, std::move(t));
    }
    cfg = c;
    for (auto& kv : loaded.tensors) tensors.add(kv.first, std::move(kv.second));
    loaded.tensors.clear();
    return true;
}
