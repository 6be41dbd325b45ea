// Loader for the reference's on-disk model directory (the MoE half of one layer): engine.idx, experts_L<l>.bin,
// nonexpert_L<l>.bin and small.bin, as written by quant/s07_pack_experts.py, s07b_pack_nonexpert.py and
// s07c_index.py, and read by the reference's Engine::load (engine/engine.cu:54-75, :166-224).
//
// engine.idx lines (quant/s07c_index.py:2-6):
//   C <key> <value>                                     config scalars
//   T <file> <name> <offset> <bytes> <dtype> <d0> [d1]  a tensor in a weight file
//   E <layer> <expert> <bits> <gu_off> <d_off>          a routed expert inside experts_L<layer>.bin (bits 0 = pruned)
//   F <file> <bytes>                                     file sizes
// The layer's routed experts come from experts_L<l>.bin, the shared expert from nonexpert_L<l>.bin (tensors
// "gate_up", "down", packlib i8 at C nonexpert_bits), the router from small.bin ("L<l>.router", bf16 [E, H]) and
// the expert bias from small.bin ("L<l>.expert_bias", fp32 [E]).
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <sstream>
#include <string>
#include <vector>

#include "llmoe.h"
#include "llmoe_internal.h"

namespace {

int lfail(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    return llmoe::set_error(LLMOE_EINVAL, buf);
}

// A stored array inside one of the model's binary files.
struct Span {
    size_t off = 0, bytes = 0;
    std::string dtype;
    std::vector<long> dims;
};

// Where one routed expert of the requested layer sits in experts_L<layer>.bin.
struct RoutedExpert {
    int bits = -1;
    long gate_up_at = -1, down_at = -1;
};

// What the loader needs from engine.idx: config scalars, every stored array (by file and name), the requested
// layer's routed experts (other layers' "E" lines are skipped) and the recorded file sizes.
struct Manifest {
    std::map<std::string, std::string> scalars;
    std::map<std::pair<std::string, std::string>, Span> spans;
    std::vector<RoutedExpert> routed;
    std::map<std::string, size_t> sizes;

    const Span* span(const std::string& file, const std::string& name) const {
        const auto it = spans.find({file, name});
        return it == spans.end() ? nullptr : &it->second;
    }
};

int parse_line(const std::string& line, int ln, int layer, Manifest& m) {
    std::istringstream s(line);
    std::string tag;
    if (!(s >> tag)) return LLMOE_OK;   // blank line
    if (tag.size() != 1) return lfail("engine.idx:%d: unknown record '%s'", ln, tag.c_str());
    switch (tag[0]) {
        case 'C': {   // C <key> <value>
            std::string key, value;
            if (!(s >> key >> value)) return lfail("engine.idx:%d: C record needs a key and a value", ln);
            m.scalars[key] = value;
            return LLMOE_OK;
        }
        case 'T': {   // T <file> <name> <offset> <bytes> <dtype> <dims...>
            std::string file, name;
            Span sp;
            if (!(s >> file >> name >> sp.off >> sp.bytes >> sp.dtype))
                return lfail("engine.idx:%d: T record needs file, name, offset, bytes, dtype", ln);
            for (long dim; s >> dim;) sp.dims.push_back(dim);
            m.spans[{file, name}] = sp;
            return LLMOE_OK;
        }
        case 'E': {   // E <layer> <expert> <bits> <gate_up offset> <down offset>
            int l = -1, e = -1;
            RoutedExpert re;
            if (!(s >> l >> e >> re.bits >> re.gate_up_at >> re.down_at) || e < 0 || e >= 65536)
                return lfail("engine.idx:%d: E record needs layer, expert (0..65535), bits, two offsets", ln);
            if (l != layer) return LLMOE_OK;
            if (size_t(e) >= m.routed.size()) m.routed.resize(size_t(e) + 1);
            m.routed[size_t(e)] = re;
            return LLMOE_OK;
        }
        case 'F': {   // F <file> <bytes>
            std::string file;
            size_t n = 0;
            if (!(s >> file >> n)) return lfail("engine.idx:%d: F record needs a file and a size", ln);
            m.sizes[file] = n;
            return LLMOE_OK;
        }
        default:
            return lfail("engine.idx:%d: unknown record '%s'", ln, tag.c_str());
    }
}

// layer < 0: no routed-expert table is collected
int read_manifest(const std::string& dir, int layer, Manifest& m) {
    std::ifstream in(dir + "/engine.idx");
    if (!in) return lfail("cannot open %s/engine.idx", dir.c_str());
    std::string line;
    for (int ln = 1; std::getline(in, line); ++ln)
        if (int rc = parse_line(line, ln, layer, m)) return rc;
    return LLMOE_OK;
}

int read_region(const std::string& path, size_t off, size_t bytes, void* dst) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) return lfail("cannot open %s", path.c_str());
    int rc = LLMOE_OK;
    if (fseeko(f, off_t(off), SEEK_SET) != 0 || fread(dst, 1, bytes, f) != bytes)
        rc = lfail("%s: cannot read %zu bytes at offset %zu", path.c_str(), bytes, off);
    fclose(f);
    return rc;
}

size_t file_bytes(const std::string& path) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) return size_t(-1);
    fseeko(f, 0, SEEK_END);
    const off_t n = ftello(f);
    fclose(f);
    return n < 0 ? size_t(-1) : size_t(n);
}

int cfg_int(const Manifest& m, const char* k, int dflt, int* out) {
    auto it = m.scalars.find(k);
    if (it == m.scalars.end()) {
        if (dflt < 0) return lfail("engine.idx: missing C %s", k);
        *out = dflt;
        return LLMOE_OK;
    }
    *out = std::atoi(it->second.c_str());
    return LLMOE_OK;
}

float bf16_to_f32(uint16_t b) {
    const uint32_t u = uint32_t(b) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

}  // namespace

extern "C" {

int llmoe_layer_load(const char* model_dir, int layer, int max_tokens, llmoe_layer** out) {
    if (!model_dir || !out) return lfail("null argument");
    *out = nullptr;
    const std::string dir(model_dir);
    Manifest ix;
    if (int rc = read_manifest(dir, layer, ix)) return rc;
    llmoe_layer_desc d{};
    int rc = cfg_int(ix, "hidden_size", -1, &d.hidden);
    if (!rc) rc = cfg_int(ix, "moe_intermediate_size", -1, &d.inter);
    if (!rc) rc = cfg_int(ix, "num_experts", -1, &d.n_experts);
    if (!rc) rc = cfg_int(ix, "num_experts_per_tok", -1, &d.top_k);
    if (!rc) rc = cfg_int(ix, "expert_capacity", 48, &d.pool);
    if (!rc) rc = cfg_int(ix, "block_size", 32, &d.block);
    int nb = 8;
    if (!rc) rc = cfg_int(ix, "nonexpert_bits", 8, &nb);
    if (rc) return rc;
    const auto rsf = ix.scalars.find("routed_scaling_factor");
    d.routed_scale = rsf != ix.scalars.end() ? float(std::atof(rsf->second.c_str())) : 2.5f;
    d.max_tokens = max_tokens;
    const int E = d.n_experts, H = d.hidden;
    if (E < 1 || E > 4096 || H < 1) return lfail("engine.idx: num_experts = %d, hidden_size = %d", E, H);
    if (int(ix.routed.size()) != E) return lfail("engine.idx: layer %d has no table of %d experts", layer, E);
    const auto& ex = ix.routed;
    const std::string exf = "experts_L" + std::to_string(layer) + ".bin";
    const std::string nef = "nonexpert_L" + std::to_string(layer) + ".bin";
    const size_t ex_bytes = file_bytes(dir + "/" + exf);
    if (ex_bytes == size_t(-1)) return lfail("cannot open %s/%s", dir.c_str(), exf.c_str());
    const auto rec = ix.sizes.find(exf);
    if (rec != ix.sizes.end() && rec->second != ex_bytes)
        return lfail("%s: %zu bytes, engine.idx says %zu", exf.c_str(), ex_bytes, rec->second);
    for (int e = 0; e < E; ++e) {
        if (ex[e].bits == 0) return lfail("layer %d expert %d is pruned (bits 0): not supported", layer, e);
        if (ex[e].bits != 2 && ex[e].bits != 3 && ex[e].bits != 4 && ex[e].bits != 8)
            return lfail("layer %d expert %d: bits = %d", layer, e, ex[e].bits);
        if (ex[e].gate_up_at < 0 || ex[e].down_at < 0) return lfail("layer %d expert %d: negative offset", layer, e);
    }
    // blob = the experts file, then (4 KiB aligned) the shared expert's gate_up and down
    const Span* gu_t = ix.span(nef, "gate_up");
    const Span* dn_t = ix.span(nef, "down");
    const bool shared = gu_t && dn_t;
    d.has_shared = shared ? 1 : 0;
    const size_t ex_pad = (ex_bytes + 4095) & ~size_t(4095);
    const size_t sh_gu = shared ? gu_t->bytes : 0, sh_dn = shared ? dn_t->bytes : 0;
    const size_t sh_dn_off = ex_pad + ((sh_gu + 4095) & ~size_t(4095));
    std::vector<uint8_t> blob(shared ? sh_dn_off + sh_dn : ex_bytes);
    if ((rc = read_region(dir + "/" + exf, 0, ex_bytes, blob.data()))) return rc;
    std::vector<uint64_t> gu_off(E + 1), d_off(E + 1);
    std::vector<int8_t> bits(E + 1);
    for (int e = 0; e < E; ++e) {
        gu_off[e] = uint64_t(ex[e].gate_up_at);
        d_off[e] = uint64_t(ex[e].down_at);
        bits[e] = int8_t(ex[e].bits);
    }
    if (shared) {
        if ((rc = read_region(dir + "/" + nef, gu_t->off, sh_gu, blob.data() + ex_pad))) return rc;
        if ((rc = read_region(dir + "/" + nef, dn_t->off, sh_dn, blob.data() + sh_dn_off))) return rc;
        gu_off[E] = ex_pad;
        d_off[E] = sh_dn_off;
        bits[E] = int8_t(nb);
    }
    // router bf16 [E, H] -> fp32 [H, E]; expert bias fp32 [E]
    const std::string pre = "L" + std::to_string(layer) + ".";
    const Span* rt = ix.span("small.bin", pre + "router");
    const Span* bt = ix.span("small.bin", pre + "expert_bias");
    if (!bt || bt->bytes != size_t(E) * 4)
        return lfail("small.bin: no fp32 [%d] L%d.expert_bias", E, layer);
    std::vector<float> bias(E), wr;
    if ((rc = read_region(dir + "/small.bin", bt->off, size_t(E) * 4, bias.data()))) return rc;
    if (rt) {
        if (rt->dtype != "bf16" || rt->bytes != size_t(E) * H * 2)
            return lfail("small.bin: L%d.router must be bf16 [%d, %d]", layer, E, H);
        std::vector<uint16_t> raw(size_t(E) * H);
        if ((rc = read_region(dir + "/small.bin", rt->off, raw.size() * 2, raw.data()))) return rc;
        wr.resize(size_t(H) * E);
        for (int e = 0; e < E; ++e)
            for (int k = 0; k < H; ++k) wr[size_t(k) * E + e] = bf16_to_f32(raw[size_t(e) * H + k]);
    }
    rc = llmoe_layer_create(&d, blob.data(), blob.size(), gu_off.data(), d_off.data(), bits.data(),
                            wr.empty() ? nullptr : wr.data(), bias.data(), out);
    return rc;
}

int llmoe_model_signs(const char* model_dir, float* signs, int n) {
    if (!model_dir || !signs) return lfail("null argument");
    Manifest ix;
    if (int rc = read_manifest(model_dir, -1, ix)) return rc;
    const Span* sp = ix.span("small.bin", "signs");
    if (!sp || sp->bytes != size_t(n) * 4) return lfail("small.bin: no fp32 [%d] signs", n);
    return read_region(std::string(model_dir) + "/small.bin", sp->off, size_t(n) * 4, signs);
}

}  // extern "C"
