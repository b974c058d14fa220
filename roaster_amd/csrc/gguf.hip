/*
 * gguf.hip -- GGUF v3 reader that fills the HBM expert table (host code only).
 *
 * Parsing follows the reference loader (weights.c:657-842): header (magic
 * "GGUF", version 3, tensor count > 0, metadata count), metadata key/value
 * pairs of which only general.alignment (uint32, non-zero; default 32) is
 * used and every other value is skipped by type (weights.c:180-244), the
 * tensor table (name, n_dims <= 4, dims, type, offset; weights.c:770-832), and
 * the data section at the first aligned position after the table
 * (weights.c:835-842).  A routed expert e of a 3-D *_exps tensor is the slice
 * [e * size / E, (e + 1) * size / E) (weights.c:380-419); since the table's
 * routed region of a kind is that tensor byte for byte, each *_exps tensor is
 * uploaded whole.  The router (blk.L.ffn_gate_inp.weight, model.c:224, F32 or
 * -- as model.c:113-121 allows -- F16 / Q4_K / Q6_K) and the shared-expert
 * gate vector (ffn_gate_inp_shexp, F32 or F16) are converted to f32 on the
 * host; the shared expert's three 2-D matrices (ffn_{gate,up,down}_shexp,
 * model.c:226-228) are uploaded as they are.  Matrix types may differ from
 * layer to layer; the table keeps them per layer.
 *
 * Unlike the reference, tensors off the MoE path are not loaded and their
 * types are not checked.
 */
#include "internal.h"
#include "table.h"

#include <stdio.h>
#include <string.h>
#include <string>
#include <vector>
#include <map>

#define GGUF_MAGIC_LE 0x46554747u        /* "GGUF" */
enum { GG_U8 = 0, GG_I8, GG_U16, GG_I16, GG_U32, GG_I32, GG_F32, GG_BOOL, GG_STR, GG_ARR, GG_U64, GG_I64, GG_F64 };
enum { GT_F32 = 0, GT_F16 = 1, GT_Q4_K = 12, GT_Q6_K = 14 };

namespace {

struct Reader {
    FILE *f = nullptr;
    uint64_t pos = 0, size = 0;
    std::string err;
    bool bad = false;
    bool read(void *dst, size_t n)
    {
        if (bad) return false;
        if (n > size - pos || fread(dst, 1, n, f) != n) {
            bad = true;
            if (err.empty()) err = "unexpected end of file at byte " + std::to_string(pos);
            return false;
        }
        pos += n;
        return true;
    }
    template <class T> bool get(T &v) { return read(&v, sizeof(v)); }
    bool skip(uint64_t n)
    {
        if (bad || n > size - pos) {
            bad = true;
            if (err.empty()) err = "unexpected end of file at byte " + std::to_string(pos);
            return false;
        }
        pos += n;
        return fseeko(f, (off_t)pos, SEEK_SET) == 0;
    }
    bool str(std::string &s)
    {
        uint64_t n;
        if (!get(n)) return false;
        if (n > size - pos || n > (1u << 20)) {
            bad = true;
            if (err.empty()) err = "string length " + std::to_string(n) + " out of range";
            return false;
        }
        s.resize((size_t)n);
        return n == 0 || read(&s[0], (size_t)n);
    }
    /* skip one metadata value of the given type (weights.c:180-244) */
    bool skip_value(uint32_t type, int depth = 0)
    {
        switch (type) {
        case GG_U8: case GG_I8: case GG_BOOL: return skip(1);
        case GG_U16: case GG_I16: return skip(2);
        case GG_U32: case GG_I32: case GG_F32: return skip(4);
        case GG_U64: case GG_I64: case GG_F64: return skip(8);
        case GG_STR: {
            uint64_t n;
            return get(n) && skip(n);
        }
        case GG_ARR: {
            uint32_t et;
            uint64_t cnt;
            if (depth > 8 || !get(et) || !get(cnt)) return false;
            const int fixed = et == GG_U8 || et == GG_I8 || et == GG_BOOL ? 1
                            : et == GG_U16 || et == GG_I16 ? 2
                            : et == GG_U32 || et == GG_I32 || et == GG_F32 ? 4
                            : et == GG_U64 || et == GG_I64 || et == GG_F64 ? 8 : 0;
            if (fixed) {
                if (cnt > (size - pos) / (uint64_t)fixed) return skip(size - pos + 1);
                return skip(cnt * (uint64_t)fixed);
            }
            for (uint64_t i = 0; i < cnt; i++)
                if (!skip_value(et, depth + 1)) return false;
            return true;
        }
        default:
            bad = true;
            err = "unknown metadata value type " + std::to_string(type);
            return false;
        }
    }
};

struct Tensor {
    std::string name;
    uint32_t n_dims = 0;
    uint64_t dims[4] = { 1, 1, 1, 1 };
    uint32_t type = 0;
    uint64_t offset = 0;
    uint64_t bytes = 0;          /* 0: a type this reader does not size */
};

uint64_t type_bytes(uint32_t type, uint64_t elements)
{
    switch (type) {
    case GT_F32: return elements * 4;
    case GT_F16: return elements * 2;
    case GT_Q4_K: return elements % 256 ? 0 : elements / 256 * RQ4K_BYTES;
    case GT_Q6_K: return elements % 256 ? 0 : elements / 256 * RQ6K_BYTES;
    default: return 0;
    }
}

/* MoE tensors of a layer, in this order */
const char *const kSuffix[8] = {
    "ffn_gate_exps.weight", "ffn_up_exps.weight", "ffn_down_exps.weight", "ffn_gate_inp.weight",
    "ffn_gate_inp_shexp.weight", "ffn_gate_shexp.weight", "ffn_up_shexp.weight", "ffn_down_shexp.weight",
};

struct Scan {
    RoasterGgufInfo info;
    std::vector<Tensor> tensors;
    std::vector<std::vector<int>> layer;     /* [L][8] tensor indices */
    std::vector<int> types;                  /* [L][6] 0 = Q4_K, 1 = Q6_K */
};

int fail_scan(const std::string &path, const std::string &why)
{
    return rt_fail(ROASTER_EINVAL, "GGUF %s: %s", path.c_str(), why.c_str());
}

int scan_file(const char *path, Scan &S, FILE **keep)
{
    memset(&S.info, 0, sizeof(S.info));
    Reader R;
    R.f = fopen(path, "rb");
    if (!R.f) return rt_fail(ROASTER_EINVAL, "GGUF %s: cannot open", path);
    if (fseeko(R.f, 0, SEEK_END) != 0) { fclose(R.f); return fail_scan(path, "cannot seek"); }
    R.size = (uint64_t)ftello(R.f);
    (void)fseeko(R.f, 0, SEEK_SET);
    auto done = [&](int rc) {
        if (rc || !keep) fclose(R.f);
        else *keep = R.f;
        return rc;
    };
    uint32_t magic = 0, version = 0;
    uint64_t n_tensors = 0, n_meta = 0;
    if (!R.get(magic) || !R.get(version) || !R.get(n_tensors) || !R.get(n_meta))
        return done(fail_scan(path, "cannot read the header"));
    if (magic != GGUF_MAGIC_LE) return done(fail_scan(path, "not a GGUF file (bad magic)"));
    if (version != 3) return done(fail_scan(path, "unsupported GGUF version " + std::to_string(version)));
    if (n_tensors == 0) return done(fail_scan(path, "no tensors"));
    if (n_tensors > (R.size >> 3) || n_meta > (R.size >> 3)) return done(fail_scan(path, "counts exceed the file size"));
    uint64_t alignment = 32;
    for (uint64_t i = 0; i < n_meta; i++) {
        std::string key;
        uint32_t type;
        if (!R.str(key) || !R.get(type)) return done(fail_scan(path, "metadata: " + R.err));
        if (key == "general.alignment" && type == GG_U32) {
            uint32_t a;
            if (!R.get(a)) return done(fail_scan(path, "metadata: " + R.err));
            if (a) alignment = a;
        } else if (!R.skip_value(type)) {
            return done(fail_scan(path, "metadata " + key + ": " + (R.err.empty() ? "truncated" : R.err)));
        }
    }
    S.tensors.resize((size_t)n_tensors);
    for (uint64_t i = 0; i < n_tensors; i++) {
        Tensor &T = S.tensors[(size_t)i];
        if (!R.str(T.name) || !R.get(T.n_dims)) return done(fail_scan(path, "tensor table: " + R.err));
        if (T.n_dims > 4) return done(fail_scan(path, "tensor " + T.name + " has more than 4 dimensions"));
        uint64_t el = 1;
        for (uint32_t d = 0; d < T.n_dims; d++) {
            if (!R.get(T.dims[d])) return done(fail_scan(path, "tensor table: " + R.err));
            if (T.dims[d] == 0 || el > UINT64_MAX / T.dims[d])
                return done(fail_scan(path, "tensor " + T.name + " has an invalid shape"));
            el *= T.dims[d];
        }
        if (!R.get(T.type) || !R.get(T.offset)) return done(fail_scan(path, "tensor table: " + R.err));
        T.bytes = type_bytes(T.type, el);
    }
    const uint64_t data = (R.pos + alignment - 1) / alignment * alignment;
    if (data > R.size) return done(fail_scan(path, "the tensor data section starts beyond the end of the file"));
    S.info.version = (int)version;
    S.info.n_tensors = n_tensors;
    S.info.alignment = alignment;
    S.info.data_offset = data;

    /* MoE tensors by layer */
    std::map<int, std::vector<int>> by_layer;
    for (size_t i = 0; i < S.tensors.size(); i++) {
        const std::string &nm = S.tensors[i].name;
        int layer = -1, used = 0;
        if (sscanf(nm.c_str(), "blk.%d.%n", &layer, &used) != 1 || used <= 0 || layer < 0 || layer > 65535) continue;
        const char *suf = nm.c_str() + used;
        for (int k = 0; k < 8; k++)
            if (!strcmp(suf, kSuffix[k])) {
                std::vector<int> &v = by_layer[layer];
                if (v.empty()) v.assign(8, -1);
                if (v[k] >= 0) return done(fail_scan(path, "duplicate tensor " + nm));
                v[k] = (int)i;
            }
    }
    if (by_layer.empty()) return done(fail_scan(path, "no MoE expert tensors (blk.N.ffn_*_exps.weight)"));
    const int n_layers = by_layer.rbegin()->first + 1;
    if ((int)by_layer.size() != n_layers)
        for (int l = 0; l < n_layers; l++)
            if (!by_layer.count(l)) return done(fail_scan(path, "layer " + std::to_string(l) + " has no MoE tensors"));
    S.layer.assign(n_layers, std::vector<int>());
    S.types.assign(6 * (size_t)n_layers, 0);
    uint64_t H = 0, I = 0, E = 0;
    for (int l = 0; l < n_layers; l++) {
        const std::vector<int> &v = by_layer[l];
        for (int k = 0; k < 8; k++)
            if (v[k] < 0)
                return done(fail_scan(path, "blk." + std::to_string(l) + "." + kSuffix[k] + " is missing"));
        const Tensor &G = S.tensors[v[0]];
        if (l == 0) { H = G.dims[0]; I = G.dims[1]; E = G.n_dims == 3 ? G.dims[2] : 0; }
        /* expected shapes: ne0 = columns (inner dimension) */
        const uint64_t want[8][3] = { { H, I, E }, { H, I, E }, { I, H, E }, { H, E, 1 },
                                      { H, 1, 1 }, { H, I, 1 }, { H, I, 1 }, { I, H, 1 } };
        const uint32_t ndim[8] = { 3, 3, 3, 2, 1, 2, 2, 2 };
        for (int k = 0; k < 8; k++) {
            const Tensor &T = S.tensors[v[k]];
            bool ok = T.n_dims == ndim[k] || (k == 4 && T.n_dims == 2 && T.dims[1] == 1);
            for (int d = 0; d < 3 && ok; d++) ok = (d < (int)T.n_dims ? T.dims[d] : 1) == want[k][d];
            if (!ok) return done(fail_scan(path, "tensor " + T.name + " has an unexpected shape"));
            const bool quant = T.type == GT_Q4_K || T.type == GT_Q6_K;
            const bool ok_type = k == 3 ? (quant || T.type == GT_F32 || T.type == GT_F16)
                               : k == 4 ? (T.type == GT_F32 || T.type == GT_F16) : quant;
            if (!ok_type || T.bytes == 0)
                return done(fail_scan(path, "tensor " + T.name + " has unsupported type " + std::to_string(T.type)));
            if (T.offset % alignment || T.offset > R.size || T.bytes > R.size - data ||
                T.offset > R.size - data - T.bytes)
                return done(fail_scan(path, "tensor " + T.name + " lies outside the file"));
            if (k <= 2) S.types[6 * (size_t)l + k] = T.type == GT_Q6_K;
            if (k >= 5) S.types[6 * (size_t)l + 3 + (k - 5)] = T.type == GT_Q6_K;
        }
        S.layer[l] = v;
        if (l == 0) S.info.router_type = (int)S.tensors[v[3]].type;
    }
    if (H == 0 || I == 0 || H % 256 || I % 256 || H > 2048 || I > 2048 || E < 8 || E > 4096)
        return done(fail_scan(path, "MoE shapes hidden " + std::to_string(H) + ", inter " + std::to_string(I) +
                                    ", experts " + std::to_string(E) + " are not supported"));
    S.info.n_layers = n_layers;
    S.info.n_experts = (int)E;
    S.info.hidden = (size_t)H;
    S.info.inter = (size_t)I;
    for (int k = 0; k < 3; k++) {
        S.info.q6[k] = S.types[k];
        S.info.sh_q6[k] = S.types[3 + k];
    }
    S.info.mixed_types = 0;
    for (int l = 1; l < n_layers; l++)
        for (int k = 0; k < 6; k++)
            if (S.types[6 * (size_t)l + k] != S.types[k]) S.info.mixed_types = 1;
    return done(0);
}

/* ---- f32 conversion of router / gate vectors (host) -------------------------- */
float half_to_float(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h >> 15) << 31, ex = (h >> 10) & 31, man = h & 1023;
    uint32_t bits;
    if (ex == 0) {
        if (man == 0) bits = sign;
        else {                               /* subnormal: man * 2^-24 */
            float f = (float)man * (1.0f / 16777216.0f);
            memcpy(&bits, &f, 4);
            bits |= sign;
        }
    } else if (ex == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((ex + 112) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* Q4_K / Q6_K super-block -> 256 f32 (GGML formats: weights w = d * sc * q -
 * dmin * m, resp. d * sc * (q - 32), kernels.c:1844-1874) */
void dequant_q4k(const uint8_t *b, float *out)
{
    const float d = half_to_float((uint16_t)(b[0] | (b[1] << 8))), dmin = half_to_float((uint16_t)(b[2] | (b[3] << 8)));
    const uint8_t *s = b + 4, *q = b + 16;
    for (int j = 0; j < 8; j++) {
        int sc, m;
        if (j < 4) { sc = s[j] & 63; m = s[j + 4] & 63; }
        else { sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4); m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4); }
        const float dl = d * (float)sc, ml = dmin * (float)m;
        for (int i = 0; i < 32; i++) {
            const int g = j >> 1, byte = q[32 * g + i];
            const int v = (j & 1) ? (byte >> 4) : (byte & 15);
            out[32 * j + i] = dl * (float)v - ml;
        }
    }
}

void dequant_q6k(const uint8_t *b, float *out)
{
    const float d = half_to_float((uint16_t)(b[208] | (b[209] << 8)));
    for (int n = 0; n < 2; n++) {
        const uint8_t *ql = b + 64 * n, *qh = b + 128 + 32 * n;
        const int8_t *sc = (const int8_t *)(b + 192 + 8 * n);
        for (int l = 0; l < 32; l++) {
            const int is = l / 16;
            const int q1 = (ql[l] & 15) | (((qh[l] >> 0) & 3) << 4);
            const int q2 = (ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4);
            const int q3 = (ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4);
            const int q4 = (ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4);
            out[128 * n + l] = d * (float)sc[is] * (float)(q1 - 32);
            out[128 * n + l + 32] = d * (float)sc[is + 2] * (float)(q2 - 32);
            out[128 * n + l + 64] = d * (float)sc[is + 4] * (float)(q3 - 32);
            out[128 * n + l + 96] = d * (float)sc[is + 6] * (float)(q4 - 32);
        }
    }
}

void to_f32(const Tensor &T, const std::vector<uint8_t> &raw, std::vector<float> &out)
{
    const uint64_t el = T.dims[0] * T.dims[1] * T.dims[2] * T.dims[3];
    out.resize((size_t)el);
    if (T.type == GT_F32) memcpy(out.data(), raw.data(), (size_t)el * 4);
    else if (T.type == GT_F16)
        for (uint64_t i = 0; i < el; i++) out[i] = half_to_float((uint16_t)(raw[2 * i] | (raw[2 * i + 1] << 8)));
    else if (T.type == GT_Q4_K)
        for (uint64_t b = 0; b < el / 256; b++) dequant_q4k(raw.data() + b * RQ4K_BYTES, out.data() + b * 256);
    else
        for (uint64_t b = 0; b < el / 256; b++) dequant_q6k(raw.data() + b * RQ6K_BYTES, out.data() + b * 256);
}

bool read_at(FILE *f, uint64_t off, uint64_t n, std::vector<uint8_t> &buf)
{
    buf.resize((size_t)n);
    return fseeko(f, (off_t)off, SEEK_SET) == 0 && fread(buf.data(), 1, (size_t)n, f) == (size_t)n;
}

}  // namespace

extern "C" int roaster_gguf_scan(const char *path, RoasterGgufInfo *info)
{
    if (!path || !info) return rt_fail(ROASTER_EINVAL, "roaster_gguf_scan: NULL argument");
    Scan S;
    const int rc = scan_file(path, S, nullptr);
    if (rc) return rc;
    *info = S.info;
    return 0;
}

extern "C" RoasterTable *roaster_table_load_gguf(const char *path, RoasterGgufInfo *info)
{
    if (!path) {
        rt_fail(ROASTER_EINVAL, "roaster_table_load_gguf: NULL path");
        return NULL;
    }
    Scan S;
    FILE *f = nullptr;
    if (scan_file(path, S, &f)) return NULL;
    RoasterTableDesc d;
    memset(&d, 0, sizeof(d));
    d.n_layers = S.info.n_layers;
    d.n_experts = S.info.n_experts;
    d.hidden = S.info.hidden;
    d.inter = S.info.inter;
    for (int k = 0; k < 3; k++) { d.q6[k] = S.info.q6[k]; d.sh_q6[k] = S.info.sh_q6[k]; }
    RoasterTable *t = roaster_table_create_layers(&d, S.types.data());
    if (!t) { fclose(f); return NULL; }
    std::vector<uint8_t> raw, sh[3];
    std::vector<float> router, gvec;
    const uint64_t base = S.info.data_offset;
    for (int l = 0; l < d.n_layers; l++) {
        const std::vector<int> &v = S.layer[l];
        for (int k = 0; k < 3; k++) {
            const Tensor &T = S.tensors[v[k]];
            if (!read_at(f, base + T.offset, T.bytes, raw)) goto io_fail;
            if (roaster_table_set_exps(t, l, k, raw.data(), raw.size())) goto fail;
        }
        {
            const Tensor &Tr = S.tensors[v[3]], &Tg = S.tensors[v[4]];
            if (!read_at(f, base + Tr.offset, Tr.bytes, raw)) goto io_fail;
            to_f32(Tr, raw, router);
            if (!read_at(f, base + Tg.offset, Tg.bytes, raw)) goto io_fail;
            to_f32(Tg, raw, gvec);
            if (roaster_table_set_router(t, l, router.data(), gvec.data())) goto fail;
        }
        for (int k = 0; k < 3; k++) {
            const Tensor &T = S.tensors[v[5 + k]];
            if (!read_at(f, base + T.offset, T.bytes, sh[k])) goto io_fail;
        }
        if (roaster_table_set_expert(t, l, d.n_experts, sh[0].data(), sh[1].data(), sh[2].data())) goto fail;
    }
    fclose(f);
    if (info) *info = S.info;
    return t;
io_fail:
    rt_fail(ROASTER_EINVAL, "GGUF %s: read error", path);
fail:
    fclose(f);
    roaster_table_destroy(t);
    return NULL;
}
