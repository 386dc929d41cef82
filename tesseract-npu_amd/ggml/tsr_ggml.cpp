// tsr_ggml.cpp -- the ggml-backend adapter over libtsr_hip (include/tsr_ggml.h): buffers, supports_op,
// lowering of a ggml graph onto the C ABI of include/tsr_hip.h, and the per-graph plan cache with HIP
// graph replay. Host code only (C++20); it reaches the device through libtsr_hip alone.
//
// What it restates from the reference backend (sw/ggml-tesseract), in its own structure:
//   - supports_op's rules (ggml-tesseract.cpp:4126-4300, tsr-build.cpp tsr_build_supports and the
//     lowering functions it probes: tsr_lower_fa :673-773, tsr_lower_rms, tsr_lower_glu, tsr_lower_rope,
//     tsr_lower_get_rows, tsr_lower_ew);
//   - the MUL_MAT lowering (ggml-tesseract.cpp:2790-2928) with its ADD / SCALE / softcap fusions
//     (tsr-build.h tsr_build_fusion: the fused node is the MUL_MAT's only user);
//   - KV-cache buffers recognized by tensor name and shape (tsr-kvbuf.h:61-63), the mask summary built
//     when the mask is written (tsr-msum.h), load-time conversion of other weight types to Q8_0
//     (tsr-weights.cpp:33-49);
//   - the plan cache keyed by graph identity (ggml-tesseract.cpp:3929-3966, 3768-3779).
// What differs by design: there is no op list to encode; a graph lowers to a list of library calls,
// and a graph that is met again replays its calls as one HIP graph (the MI355X form of the reference's
// one launch per decode token), with only the FLASH_ATTN_EXT chunk lists re-planned on the host from
// the masks of the run.
#include "tsr_ggml.h"
#include "tsr_hip.h"

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <functional>
#include <map>
#include <mutex>
#include <new>
#include <string>
#include <vector>

namespace {

constexpr uint64_t kVBase = 0x4000000000000000ull;   // buffer addresses: never dereferenced by ggml
constexpr uint64_t kVSpan = 1ull << 40;               // address space per buffer
constexpr size_t kAlign = 64;
constexpr uint32_t kKMax = 32768;                      // K_MAX (sw/sim/include/tsr_isa.h:64-67)
constexpr uint32_t kFaTMax = 680;                      // FLASH_ATTN_EXT rows per call (tsr-build.cpp:760)
constexpr size_t kShadowMax = 1u << 20;                // host copies of small index inputs
constexpr size_t kMaxPlans = 16;

enum Mode { kUndecided = 0, kLinear = 1, kWeights = 2, kKv = 3 };

struct TypeInfo {
    uint32_t blck = 0, size = 0;
    tsr_gg_to_float_fn to_float = nullptr;
    std::string name;
};

struct TInfo {                                         // a tensor init_tensor announced
    std::string name;
    uint64_t vaddr = 0;
    size_t nbytes = 0;
    int32_t type = 0;
    int64_t ne[4] = {0, 0, 0, 0};
    uint64_t nb[4] = {0, 0, 0, 0};
};

struct KvTensor {                                      // one KV-cache tensor of a KV buffer
    std::string name;
    uint64_t vaddr = 0;
    size_t nbytes = 0, row_bytes = 0;
    uint32_t which = 0, E = 0, kv_size = 0;
    int layer = -1;
    tsr_hip_kv * kv = nullptr;
};

struct Weight {                                        // a MUL_MAT weight in the library's layout
    tsr_hip_weight * w = nullptr;
    uint64_t vaddr = 0;
    size_t nbytes = 0;
    uint32_t N = 0, K = 0;
    std::vector<std::pair<uint64_t, size_t>> parts;    // a fused weight: the ggml tensors it was made of
};

struct Mask {                                          // a summarized KQ mask (written by the host)
    uint32_t n_kv = 0, n_q = 0;
    std::vector<uint16_t> f16;                         // the mask, rows of n_kv values
    std::vector<uint32_t> words;                       // its MSUM
};

struct FaSlot {                                        // one FLASH_ATTN_EXT of a plan
    tsr_hip_fa_plan * plan = nullptr;
    uint64_t mask = 0;                                 // mask data address (0: no mask)
    uint64_t kidx = 0;                                 // the K SET_ROWS indices of the same graph (0: none)
    uint32_t kidx_n = 0, T = 0, n_kv = 0;
    float scale = 0.0f;
    float * mf32 = nullptr;                            // device f32 mask copy (GENERAL summaries)
    size_t mf32_floats = 0;
    bool general = false;
    uint64_t vidx = 0;                                 // the fused form: the V SET_ROWS indices (the same cells)
    uint32_t D = 0, H = 0, Hk = 0, kv_size = 0;
};

struct Plan;
struct Call {
    tsr_gg_call info{};
    bool capturable = true;
    std::function<int(const Plan &)> run;
};

struct Plan {
    std::vector<Call> calls;
    std::vector<FaSlot> fa;
    std::vector<void *> bufs;                          // device buffers of the plan (Q|K|V rows, ROPE tables)
    bool capturable = true;
    tsr_hip_graph * graph = nullptr;
    uint64_t used = 0, runs = 0;
};

bool is_noop(int op) {
    return op == TSR_GG_OP_NONE || op == TSR_GG_OP_RESHAPE || op == TSR_GG_OP_VIEW || op == TSR_GG_OP_PERMUTE ||
           op == TSR_GG_OP_TRANSPOSE;
}

float param_f32(const tsr_gg_tensor * t, int i) {
    float f;
    memcpy(&f, &t->op_params[i], 4);
    return f;
}

int64_t nrows(const tsr_gg_tensor * t) { return t->ne[1] * t->ne[2] * t->ne[3]; }

bool same_shape(const tsr_gg_tensor * a, const tsr_gg_tensor * b) {
    return a->ne[0] == b->ne[0] && a->ne[1] == b->ne[1] && a->ne[2] == b->ne[2] && a->ne[3] == b->ne[3];
}

const tsr_gg_tensor * base_of(const tsr_gg_tensor * t) {
    while (t->view_src != nullptr) t = t->view_src;
    return t;
}

// fp32 -> fp16, round to nearest even (ggml's GGML_FP32_TO_FP16 on every host it supports).
uint16_t f2h(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);            // rounds to infinity
    if (ax < 0x38800000u) {                                               // fp16 subnormal or zero
        if (ax < 0x33000000u) return (uint16_t)sign;                      // below half the smallest
        const uint32_t e = ax >> 23, m = (ax & 0x7FFFFFu) | 0x800000u;
        const uint32_t shift = 126u - e;                                  // 14 .. 24
        uint32_t r = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (r & 1u))) ++r;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((ax >> 13) - (112u << 10));
    const uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
    return (uint16_t)(sign | r);
}

float h2f(uint16_t h) {
    const uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u;
    uint32_t u;
    if (e == 31u) u = s | 0x7F800000u | (m << 13);
    else if (e != 0u) u = s | ((e + 112u) << 23) | (m << 13);
    else if (m == 0u) u = s;
    else {
        uint32_t k = 0, mm = m;
        while ((mm & 0x400u) == 0u) { mm <<= 1; ++k; }
        u = s | ((113u - k) << 23) | ((mm & 0x3FFu) << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

float bf16f(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

// ggml's quantize_row_q8_0_ref: per 32 values d = amax / 127, id = 1/d (0 if d is 0), q = roundf(x id).
void quantize_q8_0(const float * x, int64_t K, uint8_t * out) {
    for (int64_t b = 0; b < K / 32; ++b) {
        const float * v = x + 32 * b;
        float amax = 0.0f;
        for (int j = 0; j < 32; ++j) amax = std::max(amax, std::fabs(v[j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint8_t * blk = out + 34 * b;
        const uint16_t dh = f2h(d);
        memcpy(blk, &dh, 2);
        for (int j = 0; j < 32; ++j) blk[2 + j] = (uint8_t)(int8_t)std::roundf(v[j] * id);
    }
}

uint64_t mix(uint64_t h, uint64_t v) {
    h ^= v + 0x9E3779B97F4A7C15ull + (h << 6) + (h >> 2);
    return h * 0xFF51AFD7ED558CCDull;
}

uint64_t key_tensor(uint64_t h, const tsr_gg_tensor * t) {
    h = mix(h, (uint64_t)(uint32_t)t->op << 32 | (uint32_t)t->type);
    for (int i = 0; i < 4; ++i) h = mix(mix(h, (uint64_t)t->ne[i]), t->nb[i]);
    h = mix(h, t->data);
    h = mix(h, (uint64_t)(uint32_t)t->flags);
    return h;
}

// "cache_<tag>k_l<n>" / "cache_<tag>v_l<n>" (llama.cpp's KV-cache tensor names).
bool kv_parse_name(const char * name, uint32_t * which, int * layer) {
    if (name == nullptr || strncmp(name, "cache_", 6) != 0) return false;
    const char * l = strrchr(name, '_');
    if (l == nullptr || l - name < 7 || l[1] != 'l' || l[2] == '\0') return false;
    for (const char * p = l + 2; *p; ++p)
        if (*p < '0' || *p > '9') return false;
    const char kv = l[-1];
    if (kv != 'k' && kv != 'v') return false;
    if (which) *which = kv == 'k' ? TSR_HIP_KV_K : TSR_HIP_KV_V;
    if (layer) *layer = atoi(l + 2);
    return true;
}

}  // namespace

struct tsr_gg_buffer {
    tsr_gg_dev * dev = nullptr;
    uint64_t vbase = 0;
    size_t size = 0;
    int usage = TSR_GG_USAGE_ANY;
    int mode = kUndecided;
    uint8_t * mem = nullptr;                           // device memory (kLinear, kWeights)
    std::vector<TInfo> tensors;
    std::vector<KvTensor> kv;                          // kKv, by address
};

struct tsr_gg_dev {
    int device = -1;
    tsr_hip_ctx * ctx = nullptr;
    void * stream = nullptr;
    std::recursive_mutex mtx;
    std::string err;
    std::vector<TypeInfo> foreign;
    std::vector<tsr_gg_buffer *> buffers;
    uint64_t next_vbase = kVBase;
    std::map<uint64_t, Weight> weights;                // by data address
    std::map<std::vector<uint64_t>, Weight> fused;     // concatenated / interleaved weights, by their parts
    std::map<uint64_t, Mask> masks;                    // by data address
    std::map<uint64_t, std::vector<uint8_t>> shadows;  // host copies of I32 / I64 inputs, by data address
    std::map<uint64_t, Plan> plans;
    uint64_t stamp = 0, epoch = 0;
    uint32_t options = 0;
    tsr_gg_stats st{};

    int fail(int code, const char * fmt, ...) {
        char b[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(b, sizeof b, fmt, ap);
        va_end(ap);
        err = b;
        return code;
    }
    int hip(int rc, const char * what) {
        return rc == TSR_HIP_OK ? TSR_GG_OK : fail(rc == TSR_HIP_E_NOMEM ? TSR_GG_E_NOMEM : TSR_GG_E_DEVICE,
                                                   "%s: %s", what, tsr_hip_strerror(rc));
    }
};

namespace {

bool type_info(const tsr_gg_dev * d, int32_t type, TypeInfo * out) {
    switch (type) {
        case TSR_GG_TYPE_F32: *out = {1, 4, nullptr, "f32"}; return true;
        case TSR_GG_TYPE_F16: *out = {1, 2, nullptr, "f16"}; return true;
        case TSR_GG_TYPE_BF16: *out = {1, 2, nullptr, "bf16"}; return true;
        case TSR_GG_TYPE_Q8_0: *out = {32, 34, nullptr, "q8_0"}; return true;
        case TSR_GG_TYPE_Q4_K: *out = {256, 144, nullptr, "q4_K"}; return true;
        case TSR_GG_TYPE_I32: *out = {1, 4, nullptr, "i32"}; return true;
        case TSR_GG_TYPE_I64: *out = {1, 8, nullptr, "i64"}; return true;
        default: break;
    }
    const int k = type - TSR_GG_TYPE_FOREIGN;
    if (d != nullptr && k >= 0 && k < (int)d->foreign.size()) {
        *out = d->foreign[k];
        return true;
    }
    return false;
}

size_t nbytes_of(const tsr_gg_dev * d, const tsr_gg_tensor * t) {
    TypeInfo ti;
    if (!type_info(d, t->type, &ti) || ti.blck == 0) return 0;
    size_t n = (size_t)t->ne[0] / ti.blck * ti.size;
    for (int i = 1; i < 4; ++i) n += (size_t)(t->ne[i] - 1) * t->nb[i];
    return n;
}

bool contiguous(const tsr_gg_dev * d, const tsr_gg_tensor * t) {
    TypeInfo ti;
    if (!type_info(d, t->type, &ti) || ti.blck == 0 || t->ne[0] % ti.blck != 0) return false;
    uint64_t s = ti.size;
    if (t->nb[0] != s) return false;
    s = (uint64_t)t->ne[0] / ti.blck * ti.size;
    for (int i = 1; i < 4; ++i) {
        if (t->ne[i] > 1 && t->nb[i] != s) return false;
        s *= (uint64_t)t->ne[i];
    }
    return true;
}

// A weight type the device can hold: Q8_0 / Q4_K natively, F32 / F16 / BF16 and registered types by
// conversion to Q8_0 (tsr_type_loadable, tsr-weights.cpp).
bool loadable(const tsr_gg_dev * d, int32_t type) {
    TypeInfo ti;
    if (!type_info(d, type, &ti)) return false;
    return type == TSR_GG_TYPE_Q8_0 || type == TSR_GG_TYPE_Q4_K || type == TSR_GG_TYPE_F32 || type == TSR_GG_TYPE_F16 ||
           type == TSR_GG_TYPE_BF16 || ti.to_float != nullptr;
}

tsr_gg_buffer * find_buffer(tsr_gg_dev * d, uint64_t a) {
    for (tsr_gg_buffer * b : d->buffers)
        if (a >= b->vbase && a < b->vbase + std::max<size_t>(b->size, 1)) return b;
    return nullptr;
}

bool kv_identify(const tsr_gg_dev * d, const TInfo & t, KvTensor * out, std::string * why) {
    uint32_t which = 0;
    int layer = -1;
    if (!kv_parse_name(t.name.c_str(), &which, &layer)) {
        if (why) *why = "not named cache_<tag>k_l<n> / cache_<tag>v_l<n>";
        return false;
    }
    const int64_t E = t.ne[0], cells = t.ne[1];
    if (t.type != TSR_GG_TYPE_Q8_0 || t.ne[2] != 1 || t.ne[3] != 1 || E % 64 != 0 || E < 64 || E > (int64_t)kKMax ||
        cells < 1 || cells > 0x7FFFFFFF) {
        if (why) *why = "a KV cache the device holds is q8_0 [E, kv_size, 1] with E % 64 == 0 and 64 <= E <= 32768 (one stream)";
        return false;
    }
    const size_t row = (size_t)E / 32 * 34;
    if (t.nb[0] != 34 || t.nb[1] != row) {
        if (why) *why = "the KV cache tensor is not contiguous";
        return false;
    }
    (void)d;
    out->name = t.name;
    out->vaddr = t.vaddr;
    out->nbytes = row * (size_t)cells;
    out->row_bytes = row;
    out->which = which;
    out->layer = layer;
    out->E = (uint32_t)E;
    out->kv_size = (uint32_t)cells;
    return true;
}

// The storage of a buffer, decided at its first data access: KV planes when every tensor announced is
// a KV-cache tensor, else device memory.
int decide(tsr_gg_dev * d, tsr_gg_buffer * b) {
    if (b->mode != kUndecided) return TSR_GG_OK;
    if (b->usage != TSR_GG_USAGE_WEIGHTS && !b->tensors.empty()) {
        std::vector<KvTensor> kv;
        bool all = true;
        for (const TInfo & t : b->tensors) {
            KvTensor k;
            if (!kv_identify(d, t, &k, nullptr)) { all = false; break; }
            kv.push_back(k);
        }
        if (all) {
            std::sort(kv.begin(), kv.end(), [](const KvTensor & a, const KvTensor & c) { return a.vaddr < c.vaddr; });
            for (size_t i = 1; i < kv.size(); ++i)
                if (kv[i].vaddr < kv[i - 1].vaddr + kv[i - 1].nbytes)
                    return d->fail(TSR_GG_E_ARG, "KV buffer: tensors '%s' and '%s' overlap", kv[i - 1].name.c_str(),
                                   kv[i].name.c_str());
            if (d->ctx != nullptr) {
                for (KvTensor & k : kv) {
                    const int rc = tsr_hip_kv_create(d->ctx, k.E, k.kv_size, &k.kv);
                    if (rc) {
                        for (KvTensor & f : kv) if (f.kv) tsr_hip_kv_free(d->ctx, f.kv);
                        return d->hip(rc, "KV planes");
                    }
                }
            }
            b->kv = std::move(kv);
            b->mode = kKv;
            return TSR_GG_OK;
        }
    }
    if (d->ctx != nullptr && b->size > 0) {
        void * p = nullptr;
        const int rc = tsr_hip_alloc(d->ctx, b->size, &p);
        if (rc) return d->hip(rc, "buffer memory");
        b->mem = (uint8_t *)p;
    }
    b->mode = b->usage == TSR_GG_USAGE_WEIGHTS ? kWeights : kLinear;
    return TSR_GG_OK;
}

void free_plan(tsr_gg_dev * d, Plan & p) {
    if (p.graph) tsr_hip_graph_free(d->ctx, p.graph);
    p.graph = nullptr;
    for (FaSlot & f : p.fa) {
        if (f.plan) tsr_hip_fa_plan_free(d->ctx, f.plan);
        if (f.mf32) tsr_hip_free(d->ctx, f.mf32);
        f.plan = nullptr;
        f.mf32 = nullptr;
    }
    for (void * b : p.bufs) tsr_hip_free(d->ctx, b);
    p.bufs.clear();
}

// Plans hold device pointers of weights, planes and buffers: a change to any of them empties the cache.
void drop_plans(tsr_gg_dev * d) {
    for (auto & [k, p] : d->plans) free_plan(d, p);
    d->plans.clear();
    ++d->epoch;
}

void drop_weights_in(tsr_gg_dev * d, uint64_t lo, uint64_t hi) {
    bool any = false;
    auto hit = [&](const Weight & w) {
        if (w.parts.empty()) return w.vaddr < hi && w.vaddr + w.nbytes > lo;
        for (const auto & [a, n] : w.parts)
            if (a < hi && a + n > lo) return true;
        return false;
    };
    auto sweep = [&](auto & m) {
        for (auto it = m.begin(); it != m.end();) {
            if (hit(it->second)) {
                if (!any) drop_plans(d);
                any = true;
                if (d->ctx && it->second.w) tsr_hip_weight_free(d->ctx, it->second.w);
                it = m.erase(it);
            } else {
                ++it;
            }
        }
    };
    sweep(d->weights);
    sweep(d->fused);
}

// KV buffers: byte ranges of the ggml images, across tensors.
int kv_access(tsr_gg_dev * d, tsr_gg_buffer * b, uint64_t addr, size_t n, const uint8_t * src, uint8_t * dst,
              int value) {
    uint64_t a = addr;
    const uint64_t end = addr + n;
    std::vector<uint8_t> fill;
    for (const KvTensor & k : b->kv) {
        if (a >= end) break;
        if (k.vaddr + k.nbytes <= a) continue;
        if (k.vaddr > a)
            return d->fail(TSR_GG_E_ARG, "KV buffer: bytes at 0x%llx lie between tensors", (unsigned long long)a);
        const uint64_t e = std::min<uint64_t>(end, k.vaddr + k.nbytes);
        const size_t off = a - k.vaddr, len = e - a;
        int rc;
        if (src) rc = tsr_hip_kv_set_bytes(d->ctx, k.kv, k.which, off, src + (a - addr), len);
        else if (dst) rc = tsr_hip_kv_get_bytes(d->ctx, k.kv, k.which, off, dst + (a - addr), len);
        else {
            constexpr size_t kChunk = 8u << 20;
            fill.assign(std::min(len, kChunk), (uint8_t)value);
            rc = TSR_HIP_OK;
            for (size_t o = 0; o < len && rc == TSR_HIP_OK; o += kChunk)
                rc = tsr_hip_kv_set_bytes(d->ctx, k.kv, k.which, off + o, fill.data(), std::min(kChunk, len - o));
        }
        if (rc) return d->hip(rc, k.name.c_str());
        a = e;
    }
    if (a < end) return d->fail(TSR_GG_E_ARG, "KV buffer: bytes at 0x%llx lie outside its tensors", (unsigned long long)a);
    return TSR_GG_OK;
}

// The KV tensor an address of a KV buffer falls in, with the cell.
const KvTensor * kv_at(tsr_gg_dev * d, uint64_t a, uint32_t * cell, uint32_t * byte_in_row) {
    tsr_gg_buffer * b = find_buffer(d, a);
    if (b == nullptr || decide(d, b) != TSR_GG_OK || b->mode != kKv) return nullptr;
    for (const KvTensor & k : b->kv)
        if (a >= k.vaddr && a < k.vaddr + k.nbytes) {
            *cell = (uint32_t)((a - k.vaddr) / k.row_bytes);
            *byte_in_row = (uint32_t)((a - k.vaddr) % k.row_bytes);
            return &k;
        }
    return nullptr;
}

// The KV-cache tensor a (view of a) tensor names, for supports_op before placement: its base tensor's
// announced shape (the buffer may still be undecided).
bool kv_probe(tsr_gg_dev * d, const tsr_gg_tensor * t, KvTensor * out, std::string * why) {
    const tsr_gg_tensor * bt = base_of(t);
    TInfo ti;
    ti.name = bt->name;
    ti.vaddr = bt->data;
    ti.type = bt->type;
    memcpy(ti.ne, bt->ne, sizeof ti.ne);
    memcpy(ti.nb, bt->nb, sizeof ti.nb);
    if (bt->buffer == nullptr || bt->buffer->usage == TSR_GG_USAGE_WEIGHTS) {
        if (why) *why = "not a KV-cache tensor in a buffer of this device";
        return false;
    }
    if (bt->buffer->mode != kUndecided && bt->buffer->mode != kKv) {
        if (why) *why = "its buffer holds other tensors than KV caches (device memory, not KV planes)";
        return false;
    }
    return kv_identify(d, ti, out, why);
}

// Device address of [a, a + n) in a device-memory buffer (a probe device answers the address itself).
bool dev_ptr(tsr_gg_dev * d, uint64_t a, size_t n, void ** p, std::string * why) {
    tsr_gg_buffer * b = find_buffer(d, a);
    if (b == nullptr) {
        if (why) *why = "not in a buffer of this device";
        return false;
    }
    if (decide(d, b) != TSR_GG_OK) {
        if (why) *why = d->err;
        return false;
    }
    if (b->mode != kLinear && b->mode != kWeights) {
        if (why) *why = "in a KV buffer (planes, not rows)";
        return false;
    }
    if (a + n > b->vbase + b->size) {
        if (why) *why = "extends past its buffer";
        return false;
    }
    *p = d->ctx ? (void *)(b->mem + (a - b->vbase)) : (void *)(uintptr_t)a;
    return true;
}

// Rows of f32 values: n per row, rows equally strided (floats).
struct Rows {
    uint64_t a = 0;
    void * p = nullptr;
    uint32_t n = 0, rows = 0;
    uint64_t stride = 0;
};

bool f32_rows(tsr_gg_dev * d, const tsr_gg_tensor * t, const char * what, Rows * r, std::string * why) {
    char b[256];
    if (t->type != TSR_GG_TYPE_F32 || t->nb[0] != 4 || t->nb[1] % 4 != 0) {
        snprintf(b, sizeof b, "%s '%s' is not f32 rows", what, t->name);
        *why = b;
        return false;
    }
    if ((t->ne[2] > 1 && t->nb[2] != t->nb[1] * (uint64_t)t->ne[1]) ||
        (t->ne[3] > 1 && t->nb[3] != t->nb[2] * (uint64_t)t->ne[2])) {
        snprintf(b, sizeof b, "%s '%s': its rows are not equally spaced", what, t->name);
        *why = b;
        return false;
    }
    const int64_t rr = nrows(t);
    if (t->ne[0] < 1 || rr < 1 || t->ne[0] > 0x7FFFFFFF || rr > 0x7FFFFFFF) {
        snprintf(b, sizeof b, "%s '%s' is empty or too large", what, t->name);
        *why = b;
        return false;
    }
    r->a = t->data;
    r->n = (uint32_t)t->ne[0];
    r->rows = (uint32_t)rr;
    r->stride = rr > 1 ? t->nb[1] / 4 : (uint64_t)t->ne[0];
    if (rr > 1 && r->stride < r->n) {
        snprintf(b, sizeof b, "%s '%s': rows overlap", what, t->name);
        *why = b;
        return false;
    }
    const size_t bytes = ((size_t)(r->rows - 1) * r->stride + r->n) * 4;
    std::string w2;
    if (!dev_ptr(d, r->a, bytes, &r->p, &w2)) {
        snprintf(b, sizeof b, "%s '%s' %s", what, t->name, w2.c_str());
        *why = b;
        return false;
    }
    return true;
}

// [lo, hi) of the bytes rows span
void span(const Rows & r, uint64_t * lo, uint64_t * hi) {
    *lo = r.a;
    *hi = r.a + ((uint64_t)(r.rows - 1) * r.stride + r.n) * 4;
}
bool overlap(const Rows & a, const Rows & b) {
    uint64_t l0, h0, l1, h1;
    span(a, &l0, &h0);
    span(b, &l1, &h1);
    return l0 < h1 && l1 < h0;
}
bool same_rows(const Rows & a, const Rows & b) { return a.a == b.a && a.stride == b.stride && a.n == b.n && a.rows == b.rows; }

// ---- acceptance rules ------------------------------------------------------------------------------
// A node is accepted when every requirement of its op's table holds. A table is a list of named
// predicates over a snapshot of the fields the rules read (the op's "facts", gathered once, null-safe);
// they are checked in table order and the first that fails is the refusal, reported as
//   "<OP> <rule>: <requirement> [<the facts>]"
// so that a refusal names the rule, what it asks for and what the node has.
template <class F> struct Rule {
    const char * id;                 // a short stable name of the requirement
    bool (*ok)(const F &);
    const char * need;               // what the node must have
};

std::string strf(const char * f, ...) {
    char b[512];
    va_list ap;
    va_start(ap, f);
    vsnprintf(b, sizeof b, f, ap);
    va_end(ap);
    return b;
}

template <class F, size_t N>
bool check_rules(const char * op, const F & f, const Rule<F> (&rules)[N], std::string * why) {
    for (const Rule<F> & r : rules) {
        if (r.ok(f)) continue;
        *why = strf("%s %s: %s [%s]", op, r.id, r.need, f.show().c_str());
        return false;
    }
    return true;
}

const char * type_name(int32_t t) {
    switch (t) {
        case TSR_GG_TYPE_F32: return "f32";
        case TSR_GG_TYPE_F16: return "f16";
        case TSR_GG_TYPE_BF16: return "bf16";
        case TSR_GG_TYPE_Q8_0: return "q8_0";
        case TSR_GG_TYPE_Q4_K: return "q4_K";
        case TSR_GG_TYPE_I32: return "i32";
        case TSR_GG_TYPE_I64: return "i64";
        default: return t >= TSR_GG_TYPE_FOREIGN ? "registered" : "other";
    }
}

std::string dims(const tsr_gg_tensor * t) {
    if (t == nullptr) return "none";
    return strf("'%s' %s [%lld,%lld,%lld,%lld]", t->name, type_name(t->type), (long long)t->ne[0], (long long)t->ne[1],
                (long long)t->ne[2], (long long)t->ne[3]);
}

// MUL_MAT: a weight matrix of this device times rows of f32 activations.
struct MmFacts {
    const tsr_gg_dev * d = nullptr;
    const tsr_gg_tensor * node = nullptr, * w = nullptr, * x = nullptr;
    std::string show() const { return "w " + dims(w) + ", x " + dims(x) + ", out " + dims(node); }
};
const Rule<MmFacts> kMulMatRules[] = {
    {"operands", [](const MmFacts & f) { return f.w != nullptr && f.x != nullptr; },
     "a weight matrix in src0 and activation rows in src1"},
    {"f32-io", [](const MmFacts & f) { return f.x->type == TSR_GG_TYPE_F32 && f.node->type == TSR_GG_TYPE_F32; },
     "f32 activations and an f32 result"},
    {"weight-home", [](const MmFacts & f) {
         const tsr_gg_buffer * b = base_of(f.w)->buffer;
         return b != nullptr && b->dev == f.d && b->usage != TSR_GG_USAGE_COMPUTE; },
     "src0 held by a weights (or any-usage) buffer of this device, not a compute buffer"},
    {"whole-weight", [](const MmFacts & f) {
         const tsr_gg_tensor * b = base_of(f.w);
         return f.w->view_src == nullptr || (f.w->data == b->data && same_shape(f.w, b)); },
     "src0 to be a whole weight tensor (a view covering all of it at most)"},
    {"matrix", [](const MmFacts & f) { return f.w->ne[2] == 1 && f.w->ne[3] == 1; },
     "src0 to be one 2-D matrix (ne2 = ne3 = 1)"},
    {"device-format", [](const MmFacts & f) { return loadable(f.d, f.w->type); },
     "src0 in q8_0 or q4_K, or in a type the device converts to q8_0 when it loads (f32, f16, bf16, registered)"},
    {"dense", [](const MmFacts & f) { return contiguous(f.d, f.w) && contiguous(f.d, f.x) && contiguous(f.d, f.node); },
     "contiguous src0, src1 and result"},
    {"k-range", [](const MmFacts & f) {
         const int64_t K = f.w->ne[0], N = f.w->ne[1];
         return K >= 32 && K <= (int64_t)kKMax && K % (f.w->type == TSR_GG_TYPE_Q4_K ? 256 : 32) == 0 && N >= 1 &&
                N <= 0x7FFFFFFF; },
     "32 <= K <= K_MAX (32768), K a multiple of the weight's block (32; q4_K 256), 1 <= N < 2^31"},
    {"shapes", [](const MmFacts & f) {
         return f.x->ne[0] == f.w->ne[0] && f.node->ne[0] == f.w->ne[1] && nrows(f.x) == nrows(f.node); },
     "src1 rows of K values and one result row of N values per src1 row"},
    {"x-aligned", [](const MmFacts & f) { return f.x->data % kAlign == 0; }, "src1 starting on a 64-byte boundary"},
};

// RMS_NORM: f32 rows normalized into rows of the same shape.
struct NormFacts {
    const tsr_gg_tensor * node = nullptr, * x = nullptr;
    std::string show() const { return "x " + dims(x) + ", out " + dims(node); }
};
const Rule<NormFacts> kNormRules[] = {
    {"operand", [](const NormFacts & f) { return f.x != nullptr; }, "a source"},
    {"same-shape", [](const NormFacts & f) { return same_shape(f.x, f.node) && f.node->type == TSR_GG_TYPE_F32; },
     "an f32 result of the source's shape"},
};

// ADD: a + b with b repeating whole rows of a.
struct AddFacts {
    const tsr_gg_tensor * node = nullptr, * a = nullptr, * b = nullptr;
    std::string show() const { return "a " + dims(a) + ", b " + dims(b) + ", out " + dims(node); }
};
const Rule<AddFacts> kAddRules[] = {
    {"operands", [](const AddFacts & f) { return f.a != nullptr && f.b != nullptr; }, "two sources"},
    {"same-shape", [](const AddFacts & f) { return same_shape(f.a, f.node); }, "a result of a's shape"},
};

// ROPE: rotation of f32 heads by token positions (NORMAL, NEOX and IMROPE pairings).
struct RopeFacts {
    const tsr_gg_tensor * node = nullptr, * x = nullptr, * pos = nullptr, * ff = nullptr;
    int32_t n_dims = 0, mode = 0;
    float base = 0.0f, ext = 0.0f;
    std::string show() const {
        return strf("x %s, pos %s, mode=%d n_dims=%d freq_base=%g ext_factor=%g", dims(x).c_str(), dims(pos).c_str(), mode,
                    n_dims, base, ext);
    }
    static bool heads(const tsr_gg_tensor * t, const tsr_gg_tensor * shape) {
        const uint64_t hd = (uint64_t)shape->ne[0];
        return t->type == TSR_GG_TYPE_F32 && t->nb[0] == 4 && t->nb[1] == 4 * hd && t->ne[3] == 1 &&
               (shape->ne[2] <= 1 || t->nb[2] % 4 == 0);
    }
};
const Rule<RopeFacts> kRopeRules[] = {
    {"operands", [](const RopeFacts & f) { return f.x != nullptr && f.pos != nullptr; }, "a source and positions"},
    {"mode", [](const RopeFacts & f) {
         return f.mode == TSR_HIP_ROPE_NORMAL || f.mode == TSR_HIP_ROPE_NEOX || f.mode == TSR_HIP_ROPE_IMROPE; },
     "the NORMAL, NEOX or IMROPE pairing (no multi-section or vision modes)"},
    {"no-yarn", [](const RopeFacts & f) { return f.ext == 0.0f; }, "ext_factor 0 (no YaRN extrapolation mix)"},
    {"no-offset", [](const RopeFacts & f) { return f.node->op_params[15] == 0; }, "no position offset parameter"},
    {"same-shape", [](const RopeFacts & f) { return same_shape(f.x, f.node); }, "a result of the source's shape"},
    {"f32-heads", [](const RopeFacts & f) { return RopeFacts::heads(f.x, f.node) && RopeFacts::heads(f.node, f.node); },
     "f32 source and result laid out [head_dim, n_heads, n_tokens] with each token's heads contiguous"},
    {"n-dims", [](const RopeFacts & f) {
         return f.n_dims >= 2 && f.n_dims % 2 == 0 && f.n_dims <= f.node->ne[0] && f.n_dims <= 1024; },
     "an even n_dims of at least 2 and at most head_dim (and 1024)"},
    {"positions", [](const RopeFacts & f) {
         const int64_t T = f.node->ne[2];
         return f.pos->type == TSR_GG_TYPE_I32 && f.pos->ne[0] >= (f.mode == TSR_HIP_ROPE_IMROPE ? 4 * T : T); },
     "I32 positions, one per token (four per token for IMROPE)"},
    {"imrope-positions", [](const RopeFacts & f) {
         return f.mode != TSR_HIP_ROPE_IMROPE || strstr(f.pos->name, "inp_pos") != nullptr; },
     "IMROPE positions from the graph input inp_pos (its four sections per token)"},
    {"freq-base", [](const RopeFacts & f) { return f.base > 0.0f && std::isfinite(f.base); }, "a finite positive freq_base"},
    {"freq-factors", [](const RopeFacts & f) {
         return f.ff == nullptr || (f.ff->type == TSR_GG_TYPE_F32 && f.ff->ne[0] >= f.n_dims / 2); },
     "frequency factors, when given, as an f32 vector of at least n_dims / 2"},
};

// GLU: SWIGLU of a gate and an up half (two sources, or one source of both halves).
struct GluFacts {
    const tsr_gg_tensor * node = nullptr, * g = nullptr, * u = nullptr;
    std::string show() const {
        return strf("glu op %d swapped %d, gate %s, up %s, out %s", node->op_params[0], node->op_params[1], dims(g).c_str(),
                    dims(u).c_str(), dims(node).c_str());
    }
};
const Rule<GluFacts> kGluRules[] = {
    {"swiglu", [](const GluFacts & f) { return f.node->op_params[0] == TSR_GG_GLU_SWIGLU; }, "the SWIGLU kind of GLU"},
    {"operand", [](const GluFacts & f) { return f.g != nullptr; }, "a gate source"},
    {"split-shapes", [](const GluFacts & f) { return f.u == nullptr || (same_shape(f.g, f.node) && same_shape(f.u, f.node)); },
     "gate, up and result of one shape (two-source form)"},
    {"fused-halves", [](const GluFacts & f) {
         return f.u != nullptr ||
                (f.node->op_params[1] == 0 && f.g->ne[0] == 2 * f.node->ne[0] && nrows(f.g) == nrows(f.node)); },
     "one source row of 2n values per result row of n, gate half first (one-source form)"},
};

// GET_ROWS: rows of a 2-D f32 table picked by one vector of I32 ids.
struct GetRowsFacts {
    const tsr_gg_tensor * node = nullptr, * src = nullptr, * ids = nullptr;
    std::string show() const { return "table " + dims(src) + ", ids " + dims(ids) + ", out " + dims(node); }
};
const Rule<GetRowsFacts> kGetRowsRules[] = {
    {"operands", [](const GetRowsFacts & f) { return f.src != nullptr && f.ids != nullptr; }, "a table and ids"},
    {"table", [](const GetRowsFacts & f) {
         return f.src->ne[2] == 1 && f.src->ne[3] == 1 && f.src->ne[0] == f.node->ne[0]; },
     "a 2-D table whose rows have the result's width"},
    {"ids", [](const GetRowsFacts & f) {
         return f.ids->type == TSR_GG_TYPE_I32 && f.ids->ne[1] == 1 && f.ids->ne[2] == 1; },
     "one vector of I32 ids"},
};

// SET_ROWS into one layer's KV cache (the SET_ROWS_KV kind).
struct SetRowsFacts {
    const tsr_gg_tensor * node = nullptr, * src = nullptr, * idx = nullptr;
    const tsr_gg_dev * d = nullptr;
    bool kv = false;
    std::string kv_note;
    std::string show() const {
        return "rows " + dims(src) + ", cells " + dims(idx) + ", cache " + dims(node) + (kv ? "" : " (" + kv_note + ")");
    }
};
const Rule<SetRowsFacts> kSetRowsRules[] = {
    {"operands", [](const SetRowsFacts & f) { return f.src != nullptr && f.idx != nullptr; }, "rows and cell indices"},
    {"kv-dest", [](const SetRowsFacts & f) { return f.kv; }, "a destination in a KV-cache tensor of this device"},
    {"from-cell-0", [](const SetRowsFacts & f) { return f.node->data == base_of(f.node)->data; },
     "the destination view to begin at the cache's cell 0"},
    {"i64-cells", [](const SetRowsFacts & f) {
         return f.idx->type == TSR_GG_TYPE_I64 && f.idx->ne[1] == 1 && f.idx->ne[2] == 1 && f.idx->ne[3] == 1 &&
                contiguous(f.d, f.idx); },
     "the cell indices as one contiguous I64 vector"},
};

// FLASH_ATTN_EXT: softmax attention of f32 q over one layer's q8_0 K and V planes.
struct FaFacts {
    const tsr_gg_tensor * node = nullptr, * q = nullptr, * k = nullptr, * v = nullptr, * mask = nullptr;
    float scale = 0.0f, max_bias = 0.0f, softcap = 0.0f;
    int32_t prec = 0, n_kv_max = 0;
    uint32_t D = 0, T = 0, H = 0, n_kv = 0, Hk = 0;
    bool k_kv = false, v_kv = false;
    KvTensor kk, vk;
    std::string kv_note;
    std::string show() const {
        return strf("D=%u T=%u H=%u H_kv=%u n_kv=%u scale=%g max_bias=%g softcap=%g prec=%d n_kv_max=%d; q %s, k %s, v %s, "
                    "mask %s%s%s", D, T, H, Hk, n_kv, scale, max_bias, softcap, prec, n_kv_max, dims(q).c_str(),
                    dims(k).c_str(), dims(v).c_str(), dims(mask).c_str(), kv_note.empty() ? "" : "; ", kv_note.c_str());
    }
};
const Rule<FaFacts> kFaRules[] = {
    {"operands", [](const FaFacts & f) { return f.q != nullptr && f.k != nullptr && f.v != nullptr; }, "q, K and V sources"},
    {"no-sinks", [](const FaFacts & f) { return f.node->src[4] == nullptr; }, "no attention-sink source"},
    {"plain-softmax", [](const FaFacts & f) {
         return f.max_bias == 0.0f && f.softcap == 0.0f && f.n_kv_max == 0 && (f.prec == 0 || f.prec == 10); },
     "a plain scaled softmax: no ALiBi max_bias, no logit softcap, no n_kv_max, default or F32 precision"},
    {"types", [](const FaFacts & f) {
         return f.q->type == TSR_GG_TYPE_F32 && f.k->type == TSR_GG_TYPE_Q8_0 && f.v->type == TSR_GG_TYPE_Q8_0 &&
                f.node->type == TSR_GG_TYPE_F32; },
     "q F32, K and V q8_0, an F32 result"},
    {"head-dim", [](const FaFacts & f) {
         return (f.D == 64 || f.D == 128 || f.D == 256 || f.D == 512) && f.k->ne[0] == f.D && f.v->ne[0] == f.D; },
     "one head size D for q, K and V, D in {64, 128, 256, 512}"},
    {"gqa", [](const FaFacts & f) {
         return f.Hk != 0 && f.H % f.Hk == 0 && f.H / f.Hk <= 64 && f.v->ne[1] == f.n_kv && f.v->ne[2] == f.Hk &&
                f.q->ne[3] == 1 && f.k->ne[3] == 1 && f.v->ne[3] == 1 && f.T >= 1 && f.n_kv >= 1; },
     "n_head a multiple of n_head_kv (at most 64 per KV head), V's cells and heads equal to K's, one sequence stream"},
    {"out-layout", [](const FaFacts & f) {
         return f.node->nb[0] == 4 && f.node->nb[1] == 4ull * f.D && (f.T <= 1 || f.node->nb[2] % 4 == 0) &&
                f.node->ne[0] == f.D && f.node->ne[1] == f.H && f.node->ne[2] == f.T; },
     "a result laid out [D, n_head, n_tokens] with each token's heads contiguous"},
    {"rows", [](const FaFacts & f) { return f.T <= kFaTMax; }, "at most 680 query tokens per call"},
    {"mask", [](const FaFacts & f) {
         return f.mask == nullptr || (f.mask->type == TSR_GG_TYPE_F16 && f.mask->ne[0] == f.n_kv && f.mask->ne[1] == f.T &&
                                      f.mask->ne[2] == 1 && f.mask->ne[3] == 1 && f.mask->nb[0] == 2); },
     "no mask, or an F16 mask of n_kv columns and one row per query token"},
    {"kv-views", [](const FaFacts & f) { return f.k_kv && f.v_kv; }, "K and V viewing KV-cache tensors of this device"},
    {"one-layer", [](const FaFacts & f) {
         return f.kk.which == TSR_HIP_KV_K && f.vk.which == TSR_HIP_KV_V && f.kk.E == f.Hk * f.D && f.vk.E == f.kk.E &&
                f.vk.kv_size == f.kk.kv_size; },
     "K and V as the K and V planes of one layer, E = n_head_kv D values per cell"},
    {"from-cell-0", [](const FaFacts & f) {
         const size_t cell_b = (size_t)f.kk.E / 32 * 34, head_b = (size_t)f.D / 32 * 34;
         for (const tsr_gg_tensor * t : {f.k, f.v})
             if (t->nb[0] != 34 || (f.n_kv > 1 && t->nb[1] != cell_b) || (f.Hk > 1 && t->nb[2] != head_b) ||
                 t->data != base_of(t)->data)
                 return false;
         return true; },
     "K and V views of the caches' cells from cell 0, cells a cache row apart, heads D/32 blocks apart"},
    {"fits-cache", [](const FaFacts & f) { return f.n_kv <= f.kk.kv_size; }, "n_kv no larger than the cache"},
    {"scale", [](const FaFacts & f) { return f.scale > 0.0f && std::isfinite(f.scale); }, "a finite positive scale"},
};

// The ggml rows of a weight read back from its buffer, as blocks of its device format: Q8_0 / Q4_K
// unchanged, other types to f32 and quantized to Q8_0 (ggml's quantize_row_q8_0_ref).
int weight_blocks(tsr_gg_dev * d, const tsr_gg_tensor * t, const void * p, uint32_t * fmt, std::vector<uint8_t> * out) {
    const size_t nb = nbytes_of(d, t);
    std::vector<uint8_t> raw(nb);
    const int rc = tsr_hip_read(d->ctx, raw.data(), p, nb);
    if (rc) return d->hip(rc, "weight read");
    const size_t K = (size_t)t->ne[0], N = (size_t)t->ne[1];
    if (t->type == TSR_GG_TYPE_Q4_K || t->type == TSR_GG_TYPE_Q8_0) {
        *fmt = t->type == TSR_GG_TYPE_Q4_K ? TSR_HIP_FMT_Q4_K : TSR_HIP_FMT_Q8_0;
        *out = std::move(raw);
        return TSR_GG_OK;
    }
    *fmt = TSR_HIP_FMT_Q8_0;
    TypeInfo ti;
    type_info(d, t->type, &ti);
    const size_t row_in = K / ti.blck * ti.size;
    out->assign(N * (K / 32) * 34, 0);
    std::vector<float> f(K);
    for (size_t n = 0; n < N; ++n) {
        const uint8_t * src = raw.data() + n * row_in;
        switch (t->type) {
            case TSR_GG_TYPE_F32: memcpy(f.data(), src, K * 4); break;
            case TSR_GG_TYPE_F16:
                for (size_t k = 0; k < K; ++k) { uint16_t h; memcpy(&h, src + 2 * k, 2); f[k] = h2f(h); }
                break;
            case TSR_GG_TYPE_BF16:
                for (size_t k = 0; k < K; ++k) { uint16_t h; memcpy(&h, src + 2 * k, 2); f[k] = bf16f(h); }
                break;
            default: ti.to_float(src, f.data(), (int64_t)K); break;
        }
        quantize_q8_0(f.data(), (int64_t)K, out->data() + n * (K / 32) * 34);
    }
    return TSR_GG_OK;
}

// The weight of a MUL_MAT: converted from the buffer's ggml bytes when first used.
int weight_of(tsr_gg_dev * d, const tsr_gg_tensor * t, bool build, Weight ** out, std::string * why) {
    const uint64_t a = t->data;
    auto it = d->weights.find(a);
    if (it != d->weights.end()) {
        if (it->second.N != (uint32_t)t->ne[1] || it->second.K != (uint32_t)t->ne[0]) {
            *why = "a view of a converted weight with another shape";
            return TSR_GG_E_UNSUPPORTED;
        }
        *out = &it->second;
        return TSR_GG_OK;
    }
    const size_t nb = nbytes_of(d, t);
    void * p = nullptr;
    if (!dev_ptr(d, a, nb, &p, why)) return TSR_GG_E_UNSUPPORTED;
    Weight w;
    w.vaddr = a;
    w.nbytes = nb;
    w.N = (uint32_t)t->ne[1];
    w.K = (uint32_t)t->ne[0];
    if (!build || d->ctx == nullptr) {                        // a question only: the shape, per thread
        thread_local Weight probe;
        probe = w;
        *out = &probe;
        return TSR_GG_OK;
    }
    uint32_t fmt;
    std::vector<uint8_t> blocks;
    int rc = weight_blocks(d, t, p, &fmt, &blocks);
    if (rc) return rc;
    rc = tsr_hip_weight_upload(d->ctx, fmt, blocks.data(), w.N, w.K, &w.w);
    if (rc) return d->hip(rc, "weight upload");
    d->st.weights_converted++;
    auto [ins, ok] = d->weights.emplace(a, w);
    *out = &ins->second;
    return TSR_GG_OK;
}

// The device format of a weight type: Q4_K stays Q4_K, every other type is Q8_0.
uint32_t dev_fmt(int32_t type) { return type == TSR_GG_TYPE_Q4_K ? TSR_HIP_FMT_Q4_K : TSR_HIP_FMT_Q8_0; }
size_t dev_row_bytes(uint32_t fmt, uint32_t K) { return fmt == TSR_HIP_FMT_Q4_K ? (size_t)K / 256 * 144 : (size_t)K / 32 * 34; }

// A weight made of several 2-D ggml weights of one device format and K: their rows one after another
// (Q|K|V) or, with interleave, row j of each in turn (gate / up: the library's GLU layout).
int fused_weight_of(tsr_gg_dev * d, const std::vector<const tsr_gg_tensor *> & ts, bool interleave, bool build,
                    Weight ** out, std::string * why) {
    std::vector<uint64_t> key{interleave ? 1u : 0u};
    for (const tsr_gg_tensor * t : ts) key.push_back(t->data);
    auto it = d->fused.find(key);
    if (it != d->fused.end()) {
        *out = &it->second;
        return TSR_GG_OK;
    }
    Weight w;
    w.K = (uint32_t)ts[0]->ne[0];
    const uint32_t fmt = dev_fmt(ts[0]->type);
    std::vector<void *> ps;
    for (const tsr_gg_tensor * t : ts) {
        void * p = nullptr;
        const size_t nb = nbytes_of(d, t);
        if (!dev_ptr(d, t->data, nb, &p, why)) return TSR_GG_E_UNSUPPORTED;
        ps.push_back(p);
        w.N += (uint32_t)t->ne[1];
        w.parts.emplace_back(t->data, nb);
    }
    if (!build || d->ctx == nullptr) {                        // a question only: the shape, per thread
        thread_local Weight probe;
        probe = w;
        *out = &probe;
        return TSR_GG_OK;
    }
    const size_t rb = dev_row_bytes(fmt, w.K);
    std::vector<std::vector<uint8_t>> parts(ts.size());
    for (size_t i = 0; i < ts.size(); ++i) {
        uint32_t f;
        const int rc = weight_blocks(d, ts[i], ps[i], &f, &parts[i]);
        if (rc) return rc;
    }
    std::vector<uint8_t> all((size_t)w.N * rb);
    if (interleave) {
        const size_t rows = (size_t)ts[0]->ne[1], np = ts.size();
        for (size_t r = 0; r < rows; ++r)
            for (size_t i = 0; i < np; ++i) memcpy(all.data() + (r * np + i) * rb, parts[i].data() + r * rb, rb);
    } else {
        size_t o = 0;
        for (const auto & pb : parts) {
            memcpy(all.data() + o, pb.data(), pb.size());
            o += pb.size();
        }
    }
    const int rc = tsr_hip_weight_upload(d->ctx, fmt, all.data(), w.N, w.K, &w.w);
    if (rc) return d->hip(rc, "weight upload");
    d->st.weights_converted++;
    auto [ins, ok] = d->fused.emplace(key, std::move(w));
    *out = &ins->second;
    return TSR_GG_OK;
}

// ---------------------------------------------------------------------------------------------
// Lowering
// ---------------------------------------------------------------------------------------------

struct Graph {
    const tsr_gg_tensor * const * nodes;
    int n;
    std::vector<int> uses;                              // uses of node i by later nodes
    std::vector<std::vector<int>> users;                // the later nodes that name node i as a source
    std::vector<std::pair<uint64_t, uint64_t>> out;     // bytes each node writes ([0, 0) for views)
    // some node strictly between i and j writes bytes of [lo, hi)
    bool written_between(int i, int j, uint64_t lo, uint64_t hi) const {
        for (int k = i + 1; k < j; ++k)
            if (out[k].first < hi && lo < out[k].second) return true;
        return false;
    }
    int index_of(const tsr_gg_tensor * t) const {
        for (int i = 0; i < n; ++i) if (nodes[i] == t) return i;
        return -1;
    }
    int next_real(int i) const {                        // the next node that is not a no-op
        for (int j = i + 1; j < n; ++j) if (!is_noop(nodes[j]->op)) return j;
        return -1;
    }
    bool only_user(int i, int j) const {                // node j is node i's only user, i not an output
        if (j < 0 || uses[i] != 1 || (nodes[i]->flags & TSR_GG_FLAG_OUTPUT)) return false;
        for (int s = 0; s < 10; ++s) if (nodes[j]->src[s] == nodes[i]) return true;
        return false;
    }
};

struct Lowerer {
    tsr_gg_dev * d;
    bool build;                                         // false: describe only (no device resources)
    Plan * plan;
    std::string why;
    Lowerer(tsr_gg_dev * dev, bool b, Plan * p) : d(dev), build(b), plan(p) {}
    bool fuse = true;

    void * stream() const { return d->stream; }

    Call & add(int kind, int node) {
        plan->calls.emplace_back();
        Call & c = plan->calls.back();
        c.info.kind = kind;
        c.info.node = node;
        c.info.node2 = c.info.node3 = -1;
        return c;
    }
    bool refuse(const char * fmt, ...) {
        char b[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(b, sizeof b, fmt, ap);
        va_end(ap);
        why = b;
        return false;
    }

    // MUL_MAT, with the ADD / SCALE / softcap behind it when it is their only source of this value.
    bool mul_mat(const Graph & g, int i, int * consumed) {
        const tsr_gg_tensor * node = g.nodes[i];
        MmFacts mf;
        mf.d = d;
        mf.node = node;
        mf.w = node->src[0];
        mf.x = node->src[1];
        if (!check_rules("MUL_MAT", mf, kMulMatRules, &why)) return false;
        const tsr_gg_tensor * w = mf.w;
        const tsr_gg_tensor * x = mf.x;
        const int64_t K = w->ne[0], N = w->ne[1];
        // src1 = RMS_NORM(x') * w folded into this matvec: the norm runs on x' inside it
        const int xi = g.index_of(x);
        const Fold * fo = xi >= 0 && xi < (int)fold_of.size() && fold_of[xi] >= 0 ? &folds[fold_of[xi]] : nullptr;
        Rows X, Y, NW;
        if (!f32_rows(d, fo ? fo->x : x, "src1", &X, &why)) return false;
        if (fo && !f32_rows(d, fo->w, "norm weight", &NW, &why)) return false;
        Weight * wt = nullptr;
        int rc = weight_of(d, w, build, &wt, &why);
        if (rc) {
            if (rc != TSR_GG_E_UNSUPPORTED) why = d->err;
            return false;
        }
        const uint32_t T = X.rows;
        // the fused consumer: ADD of an f32 addend (same shape, or one row), SCALE, or SCALE-TANH-SCALE
        const tsr_gg_tensor * out = node;
        const tsr_gg_tensor * addend = nullptr;
        uint32_t flags = 0;
        float s1 = 0.0f, s2 = 0.0f;
        int n2 = -1, n3 = -1, last = i;
        const int u = fuse ? g.next_real(i) : -1;
        if (u >= 0 && g.only_user(i, u) && !skip[u]) {
            const tsr_gg_tensor * un = g.nodes[u];
            if (fo && un->op == TSR_GG_OP_SCALE) {
                // the norm form has no epilogue: never reached (a fold is refused for such readers)
            } else if (un->op == TSR_GG_OP_ADD && same_shape(un, node) && un->type == TSR_GG_TYPE_F32) {
                const tsr_gg_tensor * o = un->src[0] == node ? un->src[1] : un->src[0];
                if (o != nullptr && o != node && o->type == TSR_GG_TYPE_F32 && o->ne[0] == N &&
                    (nrows(o) == 1 || same_shape(o, node))) {
                    out = un;
                    addend = o;
                    n2 = last = u;
                }
            } else if (un->op == TSR_GG_OP_SCALE && param_f32(un, 1) == 0.0f && same_shape(un, node)) {
                const int v = g.next_real(u);
                const tsr_gg_tensor * vn = v >= 0 ? g.nodes[v] : nullptr;
                const int z = v >= 0 ? g.next_real(v) : -1;
                const tsr_gg_tensor * zn = z >= 0 ? g.nodes[z] : nullptr;
                if (vn && zn && vn->op == TSR_GG_OP_UNARY && vn->op_params[0] == TSR_GG_UNARY_TANH && g.only_user(u, v) &&
                    zn->op == TSR_GG_OP_SCALE && param_f32(zn, 1) == 0.0f && g.only_user(v, z) && same_shape(zn, node)) {
                    out = zn;
                    flags = TSR_HIP_MM_SOFTCAP;
                    s1 = param_f32(un, 0);
                    s2 = param_f32(zn, 0);
                    n2 = u;
                    n3 = z;
                    last = z;
                } else {
                    out = un;
                    flags = TSR_HIP_MM_SCALE;
                    s2 = param_f32(un, 0);
                    n2 = last = u;
                }
            }
        }
        if (!f32_rows(d, out, "dst", &Y, &why)) return false;
        Rows A;
        if (addend != nullptr) {
            if (!f32_rows(d, addend, "addend", &A, &why)) return false;
            if (overlap(A, Y) && !same_rows(A, Y)) { addend = nullptr; out = node; n2 = -1; last = i; }
            else if (overlap(X, Y)) { addend = nullptr; out = node; n2 = -1; last = i; }
            if (addend == nullptr && !f32_rows(d, node, "dst", &Y, &why)) return false;
        } else if (out != node && overlap(X, Y)) {
            out = node;
            flags = 0;
            n2 = n3 = -1;
            last = i;
            if (!f32_rows(d, node, "dst", &Y, &why)) return false;
        }
        if (overlap(X, Y)) return refuse("MUL_MAT in-place: the result may not share bytes with src1");
        Call & c = add(TSR_GG_CALL_MUL_MAT, i);
        c.info.node2 = n2;
        c.info.node3 = n3;
        c.info.N = (uint32_t)N;
        c.info.K = (uint32_t)K;
        c.info.T = T;
        c.info.flags = flags;
        c.info.x = X.a;
        c.info.y = Y.a;
        c.info.add = addend ? A.a : 0;
        c.info.w = w->data;
        c.info.x_stride = X.stride;
        c.info.y_stride = Y.stride;
        c.info.add_stride = addend ? (A.rows == 1 ? 0 : A.stride) : 0;
        c.info.scale = s1;
        c.info.scale2 = s2;
        if (fo) {
            c.info.node3 = fo->norm;
            c.info.scale = fo->eps;
        }
        c.capturable = T < 16;
        if (build) {
            tsr_hip_ctx * ctx = d->ctx;
            const tsr_hip_weight * hw = wt->w;
            const float * xp = (const float *)X.p;
            float * yp = (float *)Y.p;
            const float * ap = addend ? (const float *)A.p : nullptr;
            const uint64_t xs = X.stride, ys = Y.stride, as = c.info.add_stride;
            void * s = stream();
            if (fo) {
                const float eps = fo->eps;
                const float * nw = (const float *)NW.p;
                c.run = [=](const Plan &) { return tsr_hip_mul_mat_norm(ctx, hw, xp, T, xs, eps, nw, yp, ys, ap, as, 0u, s); };
            } else if (flags) {
                c.run = [=](const Plan &) { return tsr_hip_mul_mat_epi(ctx, hw, xp, T, xs, yp, ys, ap, as, flags, s1, s2, s); };
            } else {
                c.run = [=](const Plan &) { return tsr_hip_mul_mat(ctx, hw, xp, T, xs, yp, ys, ap, as, 0u, s); };
            }
        }
        *consumed = last;
        return true;
    }

    // The ROPE acceptance rules of a node (also of the q rotation a fused attention call performs).
    bool rope_rules(const tsr_gg_tensor * node, RopeFacts * rf) {
        rf->node = node;
        rf->x = node->src[0];
        rf->pos = node->src[1];
        rf->ff = node->src[2];
        rf->n_dims = node->op_params[1];
        rf->mode = node->op_params[2];
        rf->base = param_f32(node, 5);
        rf->ext = param_f32(node, 7);
        return check_rules("ROPE", *rf, kRopeRules, &why);
    }

    // RMS_NORM, with the MUL by a weight row behind it when it is the norm's only user.
    bool rms_norm(const Graph & g, int i, int * consumed) {
        const tsr_gg_tensor * node = g.nodes[i];
        NormFacts nf;
        nf.node = node;
        nf.x = node->src[0];
        if (!check_rules("RMS_NORM", nf, kNormRules, &why)) return false;
        const tsr_gg_tensor * x = nf.x;
        Rows X, Y, W;
        if (!f32_rows(d, x, "source", &X, &why)) return false;
        const tsr_gg_tensor * out = node;
        const tsr_gg_tensor * wt = nullptr;
        int n2 = -1;
        const int u = g.next_real(i);
        if (u >= 0 && g.only_user(i, u) && g.nodes[u]->op == TSR_GG_OP_MUL && same_shape(g.nodes[u], node)) {
            // RMS_NORM + MUL is one record in every lowering (a MUL by a weight has no call of its own)
            const tsr_gg_tensor * un = g.nodes[u];
            const tsr_gg_tensor * o = un->src[0] == node ? un->src[1] : un->src[0];
            if (o && o->type == TSR_GG_TYPE_F32 && o->ne[0] == node->ne[0] && (nrows(o) == 1 || nrows(o) == nrows(node))) {
                out = un;
                wt = o;
                n2 = u;
            }
        }
        if (!f32_rows(d, out, "result", &Y, &why)) return false;
        if (wt && !f32_rows(d, wt, "weight", &W, &why)) return false;
        if (overlap(X, Y) && !same_rows(X, Y)) return refuse("RMS_NORM in-place: the result is the source itself or apart from it");
        Call & c = add(TSR_GG_CALL_RMS_NORM, i);
        c.info.node2 = n2;
        c.info.N = X.n;
        c.info.T = X.rows;
        c.info.x = X.a;
        c.info.y = Y.a;
        c.info.w = wt ? W.a : 0;
        c.info.x_stride = X.stride;
        c.info.y_stride = Y.stride;
        c.info.add_stride = wt ? W.stride : 0;
        c.info.scale = param_f32(node, 0);
        if (build) {
            tsr_hip_ctx * ctx = d->ctx;
            const float * xp = (const float *)X.p;
            float * yp = (float *)Y.p;
            const float * wp = wt ? (const float *)W.p : nullptr;
            const uint32_t n = X.n, rows = X.rows, wper = wt ? W.rows : 1;
            const uint64_t xs = X.stride, ys = Y.stride, ws = wt ? W.stride : 0;
            const float eps = c.info.scale;
            void * s = stream();
            c.run = [=](const Plan &) { return tsr_hip_rms_norm(ctx, xp, n, rows, xs, eps, wp, ws, wper, yp, ys, s); };
        }
        *consumed = n2 >= 0 ? n2 : i;
        return true;
    }

    bool add_op(const Graph & g, int i) {
        const tsr_gg_tensor * node = g.nodes[i];
        AddFacts af;
        af.node = node;
        af.a = node->src[0];
        af.b = node->src[1];
        if (!check_rules("ADD", af, kAddRules, &why)) return false;
        const tsr_gg_tensor * a = af.a;
        const tsr_gg_tensor * b = af.b;
        Rows A, B, Y;
        if (!f32_rows(d, a, "a", &A, &why) || !f32_rows(d, b, "b", &B, &why) || !f32_rows(d, node, "result", &Y, &why))
            return false;
        // b repeats: one row for all, or every row, or (2-D results) a period of whole rows
        const bool whole_rows = B.n == Y.n && (B.rows == 1 || B.rows == Y.rows ||
                                               (Y.rows % B.rows == 0 && node->ne[2] <= 1 && node->ne[3] <= 1));
        if (!whole_rows)
            return refuse("ADD row-broadcast: b must repeat whole rows of the result [%s]", af.show().c_str());
        if ((overlap(A, Y) && !same_rows(A, Y)) || (overlap(B, Y) && !same_rows(B, Y)))
            return refuse("ADD in-place: the result is an operand itself or apart from both");
        Call & c = add(TSR_GG_CALL_ADD, i);
        c.info.N = Y.n;
        c.info.T = Y.rows;
        c.info.x = A.a;
        c.info.add = B.a;
        c.info.y = Y.a;
        c.info.x_stride = A.stride;
        c.info.add_stride = B.stride;
        c.info.y_stride = Y.stride;
        if (build) {
            tsr_hip_ctx * ctx = d->ctx;
            const float * ap = (const float *)A.p;
            const float * bp = (const float *)B.p;
            float * yp = (float *)Y.p;
            const uint64_t as = A.stride, bs = B.stride, ys = Y.stride;
            const uint32_t per = B.rows, n = Y.n, rows = Y.rows;
            void * s = stream();
            c.run = [=](const Plan &) { return tsr_hip_add(ctx, ap, as, bp, bs, per, n, rows, yp, ys, s); };
        }
        return true;
    }

    bool rope(const Graph & g, int i) {
        const tsr_gg_tensor * node = g.nodes[i];
        RopeFacts rf;
        if (!rope_rules(node, &rf)) return false;
        const tsr_gg_tensor * x = rf.x;
        const tsr_gg_tensor * pos = rf.pos;
        const tsr_gg_tensor * ff = rf.ff;
        const int32_t n_dims = rf.n_dims, mode = rf.mode;
        const float freq_base = rf.base, freq_scale = param_f32(node, 6), attn = param_f32(node, 8);
        const uint32_t hd = (uint32_t)node->ne[0], nh = (uint32_t)node->ne[1], T = (uint32_t)node->ne[2];
        const uint64_t xs = T > 1 ? x->nb[2] / 4 : (uint64_t)hd * nh, ys = T > 1 ? node->nb[2] / 4 : (uint64_t)hd * nh;
        void *xp, *yp, *pp, *fp = nullptr;
        const size_t xb = ((size_t)(T - 1) * xs + (size_t)hd * nh) * 4, yb = ((size_t)(T - 1) * ys + (size_t)hd * nh) * 4;
        std::string w2;
        if (!dev_ptr(d, x->data, xb, &xp, &w2) || !dev_ptr(d, node->data, yb, &yp, &w2) ||
            !dev_ptr(d, pos->data, 4 * (size_t)pos->ne[0], &pp, &w2))
            return refuse("ROPE device-rows: source, result and positions in device memory of this device (%s)", w2.c_str());
        if (ff != nullptr) {
            if (!contiguous(d, ff) || !dev_ptr(d, ff->data, 4 * (size_t)ff->ne[0], &fp, &w2))
                return refuse("ROPE freq-factors: a contiguous vector in device memory of this device (%s)", w2.c_str());
        }
        if (x->data != node->data && x->data < node->data + yb && node->data < x->data + xb)
            return refuse("ROPE in-place: the result is the source itself or apart from it");
        Call & c = add(TSR_GG_CALL_ROPE, i);
        c.info.N = hd;
        c.info.K = nh;
        c.info.T = T;
        c.info.x = x->data;
        c.info.y = node->data;
        c.info.add = pos->data;
        c.info.w = ff ? ff->data : 0;
        c.info.x_stride = xs;
        c.info.y_stride = ys;
        c.info.mode = (uint32_t)mode;
        c.info.n_dims = (uint32_t)n_dims;
        c.info.scale = freq_base;
        c.info.scale2 = attn;
        if (build) {
            tsr_hip_ctx * ctx = d->ctx;
            void * s = stream();
            const uint32_t nd = (uint32_t)n_dims;
            c.run = [=](const Plan &) {
                return tsr_hip_rope(ctx, (const float *)xp, T, xs, hd, nh, nd, mode, (const int32_t *)pp, freq_base, freq_scale,
                                    attn, (const float *)fp, (float *)yp, ys, s);
            };
        }
        return true;
    }

    bool glu(const Graph & g, int i) {
        const tsr_gg_tensor * node = g.nodes[i];
        GluFacts gf;
        gf.node = node;
        gf.g = node->src[0];
        gf.u = node->src[1];
        if (!check_rules("GLU", gf, kGluRules, &why)) return false;
        const tsr_gg_tensor * gt = gf.g;
        const tsr_gg_tensor * ut = gf.u;
        Rows G, U, Y;
        if (!f32_rows(d, node, "result", &Y, &why)) return false;
        if (ut != nullptr) {
            if (!f32_rows(d, gt, "gate", &G, &why) || !f32_rows(d, ut, "up", &U, &why)) return false;
        } else {
            if (!f32_rows(d, gt, "gate|up", &G, &why)) return false;
            U = G;
            U.a += 4ull * (uint64_t)node->ne[0];
            U.p = d->ctx ? (void *)((uint8_t *)G.p + 4 * node->ne[0]) : (void *)(uintptr_t)U.a;
            G.n = U.n = (uint32_t)node->ne[0];
        }
        if ((overlap(G, Y) && !same_rows(G, Y)) || (overlap(U, Y) && !same_rows(U, Y)))
            return refuse("GLU in-place: the result is a source itself or apart from both");
        Call & c = add(TSR_GG_CALL_SWIGLU, i);
        c.info.N = Y.n;
        c.info.T = Y.rows;
        c.info.x = G.a;
        c.info.add = U.a;
        c.info.y = Y.a;
        c.info.x_stride = G.stride;
        c.info.add_stride = U.stride;
        c.info.y_stride = Y.stride;
        if (build) {
            tsr_hip_ctx * ctx = d->ctx;
            const float * gp = (const float *)G.p;
            const float * up = (const float *)U.p;
            float * yp = (float *)Y.p;
            const uint64_t gs = G.stride, us = U.stride, ys = Y.stride;
            const uint32_t n = Y.n, rows = Y.rows;
            void * s = stream();
            c.run = [=](const Plan &) { return tsr_hip_swiglu(ctx, gp, gs, up, us, n, rows, yp, ys, s); };
        }
        return true;
    }

    bool get_rows(const Graph & g, int i) {
        const tsr_gg_tensor * node = g.nodes[i];
        GetRowsFacts gf;
        gf.node = node;
        gf.src = node->src[0];
        gf.ids = node->src[1];
        if (!check_rules("GET_ROWS", gf, kGetRowsRules, &why)) return false;
        const tsr_gg_tensor * src = gf.src;
        const tsr_gg_tensor * ids = gf.ids;
        Rows S, Y;
        if (!f32_rows(d, src, "table", &S, &why) || !f32_rows(d, node, "result", &Y, &why)) return false;
        void * ip = nullptr;
        std::string w2;
        if (!dev_ptr(d, ids->data, 4 * (size_t)ids->ne[0], &ip, &w2))
            return refuse("GET_ROWS device-ids: the ids in device memory of this device (%s)", w2.c_str());
        if (overlap(S, Y)) return refuse("GET_ROWS in-place: the result may not share bytes with the table");
        Call & c = add(TSR_GG_CALL_GET_ROWS, i);
        c.info.N = S.n;
        c.info.K = S.rows;
        c.info.T = (uint32_t)ids->ne[0];
        c.info.w = S.a;
        c.info.x = ids->data;
        c.info.y = Y.a;
        c.info.x_stride = S.stride;
        c.info.y_stride = Y.stride;
        if (build) {
            tsr_hip_ctx * ctx = d->ctx;
            const float * sp = (const float *)S.p;
            float * yp = (float *)Y.p;
            const uint64_t ss = S.stride, ys = Y.stride;
            const uint32_t n = S.n, n_src = S.rows, cnt = c.info.T;
            void * s = stream();
            c.run = [=](const Plan &) { return tsr_hip_get_rows(ctx, sp, ss, n, n_src, (const int32_t *)ip, cnt, yp, ys, nullptr, s); };
        }
        return true;
    }

    bool argmax(const Graph & g, int i) {
        const tsr_gg_tensor * node = g.nodes[i];
        const tsr_gg_tensor * x = node->src[0];
        Rows X;
        if (x == nullptr) return refuse("ARGMAX operand: a source of f32 rows [none]");
        if (!f32_rows(d, x, "source", &X, &why)) return false;
        if (node->type != TSR_GG_TYPE_I32 || node->ne[0] != (int64_t)X.rows || !contiguous(d, node))
            return refuse("ARGMAX i32-index: one contiguous I32 index per source row [out %s]", dims(node).c_str());
        void * yp = nullptr;
        std::string w2;
        if (!dev_ptr(d, node->data, 4ull * X.rows, &yp, &w2))
            return refuse("ARGMAX device-rows: the result in device memory of this device (%s)", w2.c_str());
        Call & c = add(TSR_GG_CALL_ARGMAX, i);
        c.info.N = X.n;
        c.info.T = X.rows;
        c.info.x = X.a;
        c.info.y = node->data;
        c.info.x_stride = X.stride;
        if (build) {
            tsr_hip_ctx * ctx = d->ctx;
            const float * xp = (const float *)X.p;
            const uint32_t n = X.n, rows = X.rows;
            const uint64_t xs = X.stride;
            void * s = stream();
            c.run = [=](const Plan &) { return tsr_hip_argmax(ctx, xp, n, rows, xs, (int32_t *)yp, s); };
        }
        return true;
    }

    // SET_ROWS into a KV-cache tensor (the SET_ROWS_KV kind).
    bool set_rows(const Graph & g, int i) {
        const tsr_gg_tensor * node = g.nodes[i];
        SetRowsFacts sf;
        sf.d = d;
        sf.node = node;
        sf.src = node->src[0];
        sf.idx = node->src[1];
        KvTensor kp;
        sf.kv = kv_probe(d, node, &kp, &sf.kv_note);
        if (!check_rules("SET_ROWS", sf, kSetRowsRules, &why)) return false;
        const tsr_gg_tensor * src = sf.src;
        const tsr_gg_tensor * idx = sf.idx;
        Rows S;
        if (!f32_rows(d, src, "rows", &S, &why)) return false;
        if (S.n != kp.E || (int64_t)S.rows != idx->ne[0])
            return refuse("SET_ROWS row-width: one source row of E = %u values per cell index [%s]", kp.E, sf.show().c_str());
        void * ip = nullptr;
        std::string w2;
        if (!dev_ptr(d, idx->data, 8 * (size_t)idx->ne[0], &ip, &w2))
            return refuse("SET_ROWS device-cells: the cell indices in device memory of this device (%s)", w2.c_str());
        Call & c = add(TSR_GG_CALL_SET_ROWS, i);
        c.info.N = S.n;
        c.info.T = S.rows;
        c.info.x = S.a;
        c.info.add = idx->data;
        c.info.y = node->data;
        c.info.x_stride = S.stride;
        c.info.which = kp.which;
        c.info.kv_size = kp.kv_size;
        if (build) {
            uint32_t cell, bir;
            const KvTensor * k = kv_at(d, base_of(node)->data, &cell, &bir);
            if (k == nullptr) return refuse("SET_ROWS: the KV cache is not placed");
            tsr_hip_ctx * ctx = d->ctx;
            tsr_hip_kv * kv = k->kv;
            const uint32_t which = k->which, n_rows = S.rows;
            const float * sp = (const float *)S.p;
            const uint64_t ss = S.stride;
            void * s = stream();
            c.run = [=](const Plan &) { return tsr_hip_kv_set_rows(ctx, kv, which, sp, n_rows, ss, (const int64_t *)ip, nullptr, s); };
        }
        return true;
    }

    // FLASH_ATTN_EXT over one layer's K and V planes (tsr_lower_fa, tsr-build.cpp:673-773): the rules of
    // everything but q, the result and the new cells.
    struct FaInfo {
        uint32_t D = 0, T = 0, H = 0, Hk = 0, n_kv = 0, kv_size = 0;
        float scale = 0.0f;
        uint64_t mask = 0, kidx = 0, kbase = 0, vbase = 0;
        uint32_t kidx_n = 0;
        void * op = nullptr;
        uint64_t os = 0;
    };
    bool fa_info(const Graph & g, int i, FaInfo * f) {
        const tsr_gg_tensor * node = g.nodes[i];
        FaFacts ff;
        ff.node = node;
        ff.q = node->src[0];
        ff.k = node->src[1];
        ff.v = node->src[2];
        ff.mask = node->src[3];
        ff.scale = param_f32(node, 0);
        ff.max_bias = param_f32(node, 1);
        ff.softcap = param_f32(node, 2);
        ff.prec = node->op_params[3];
        ff.n_kv_max = node->op_params[4];
        if (ff.q != nullptr && ff.k != nullptr && ff.v != nullptr) {
            ff.D = (uint32_t)ff.q->ne[0];
            ff.T = (uint32_t)ff.q->ne[1];
            ff.H = (uint32_t)ff.q->ne[2];
            ff.n_kv = (uint32_t)ff.k->ne[1];
            ff.Hk = (uint32_t)ff.k->ne[2];
            std::string kn, vn;
            ff.k_kv = kv_probe(d, ff.k, &ff.kk, &kn);
            ff.v_kv = kv_probe(d, ff.v, &ff.vk, &vn);
            if (!ff.k_kv) ff.kv_note = "K: " + kn;
            if (!ff.v_kv) ff.kv_note += std::string(ff.kv_note.empty() ? "" : "; ") + "V: " + vn;
        }
        if (!check_rules("FLASH_ATTN_EXT", ff, kFaRules, &why)) return false;
        const tsr_gg_tensor * k = ff.k;
        const uint32_t D = ff.D, T = ff.T, H = ff.H;
        f->os = T > 1 ? node->nb[2] / 4 : (uint64_t)H * D;
        std::string w2;
        if (!dev_ptr(d, node->data, ((size_t)(T - 1) * f->os + (size_t)H * D) * 4, &f->op, &w2))
            return refuse("FLASH_ATTN_EXT device-rows: the result in device memory of this device (%s)", w2.c_str());
        // the new cells: the indices of an earlier SET_ROWS of this graph into the same K cache, which the
        // host writes (their copy on the host orders the chunk plan: the newest cells last)
        for (int j = 0; j < i; ++j) {
            const tsr_gg_tensor * sj = g.nodes[j];
            if (sj->op != TSR_GG_OP_SET_ROWS || base_of(sj)->data != base_of(k)->data || sj->src[1] == nullptr) continue;
            const tsr_gg_tensor * ix = sj->src[1];
            if (ix->op != TSR_GG_OP_NONE || g.index_of(ix) >= 0)
                return refuse("FLASH_ATTN_EXT host-cells: new-cell indices the host writes, not a result of the graph [%s]",
                              dims(ix).c_str());
            f->kidx = ix->data;
            f->kidx_n = (uint32_t)ix->ne[0];
        }
        f->D = D;
        f->T = T;
        f->H = H;
        f->Hk = ff.Hk;
        f->n_kv = ff.n_kv;
        f->kv_size = ff.kk.kv_size;
        f->scale = ff.scale;
        f->mask = ff.mask ? ff.mask->data : 0;
        f->kbase = base_of(k)->data;
        f->vbase = base_of(ff.v)->data;
        return true;
    }
    void fa_call_info(Call & c, const FaInfo & f, uint64_t q, uint64_t qs, uint64_t y) {
        c.info.D = f.D;
        c.info.n_head = f.H;
        c.info.n_head_kv = f.Hk;
        c.info.n_kv = f.n_kv;
        c.info.kv_size = f.kv_size;
        c.info.T = f.T;
        c.info.x = q;
        c.info.y = y;
        c.info.add = f.mask;
        c.info.w = f.kidx;
        c.info.x_stride = qs;
        c.info.y_stride = f.os;
        c.info.scale = f.scale;
        c.info.K = f.kidx_n;
    }
    // The plan of a FLASH_ATTN_EXT (build mode): one per shape, mask and new cells, shared by the layers
    // of a graph (their launches run one after another on one stream). -1 on failure (why set).
    int fa_slot(const FaInfo & f, uint64_t vidx) {
        for (size_t i = 0; i < plan->fa.size(); ++i) {
            const FaSlot & s = plan->fa[i];
            if (s.mask == f.mask && s.kidx == f.kidx && s.vidx == vidx && s.kidx_n == f.kidx_n && s.T == f.T &&
                s.n_kv == f.n_kv && s.scale == f.scale && s.D == f.D && s.H == f.H && s.Hk == f.Hk && s.kv_size == f.kv_size)
                return (int)i;
        }
        FaSlot s;
        const int rc = tsr_hip_fa_plan_create(d->ctx, f.D, f.H, f.Hk, f.T, f.kv_size, &s.plan);
        if (rc) {
            why = std::string("FA plan: ") + tsr_hip_strerror(rc);
            return -1;
        }
        s.mask = f.mask;
        s.kidx = f.kidx;
        s.vidx = vidx;
        s.kidx_n = f.kidx_n;
        s.T = f.T;
        s.n_kv = f.n_kv;
        s.scale = f.scale;
        s.D = f.D;
        s.H = f.H;
        s.Hk = f.Hk;
        s.kv_size = f.kv_size;
        s.mf32_floats = (size_t)f.T * 16u * ((f.n_kv + 15u) / 16u);
        plan->fa.push_back(s);
        return (int)plan->fa.size() - 1;
    }
    bool flash_attn(const Graph & g, int i) {
        FaInfo f;
        if (!fa_info(g, i, &f)) return false;
        const tsr_gg_tensor * q = g.nodes[i]->src[0];
        if (q->nb[0] != 4 || q->nb[2] != 4ull * f.D || (f.T > 1 && q->nb[1] % 4 != 0))
            return refuse("FLASH_ATTN_EXT q-rows: each token's q heads contiguous, D floats apart [q %s]", dims(q).c_str());
        const uint64_t qs = f.T > 1 ? q->nb[1] / 4 : (uint64_t)f.H * f.D;
        void * qp = nullptr;
        std::string w2;
        if (!dev_ptr(d, q->data, ((size_t)(f.T - 1) * qs + (size_t)f.H * f.D) * 4, &qp, &w2))
            return refuse("FLASH_ATTN_EXT device-q: q in device memory of this device (%s)", w2.c_str());
        Call & c = add(TSR_GG_CALL_FLASH_ATTN, i);
        fa_call_info(c, f, q->data, qs, g.nodes[i]->data);
        if (build) {
            uint32_t cell, bir;
            const KvTensor * kt = kv_at(d, f.kbase, &cell, &bir);
            const KvTensor * vt = kv_at(d, f.vbase, &cell, &bir);
            if (kt == nullptr || vt == nullptr) return refuse("FLASH_ATTN_EXT: the KV caches are not placed");
            const int slot = fa_slot(f, 0);
            if (slot < 0) return false;
            tsr_hip_ctx * ctx = d->ctx;
            const tsr_hip_kv * kc = kt->kv;
            const tsr_hip_kv * vc = vt->kv;
            void * s = stream();
            void * op = f.op;
            const uint64_t os = f.os;
            const float scale = f.scale;
            c.run = [=](const Plan & pl) {
                const FaSlot & fs = pl.fa[slot];
                return tsr_hip_flash_attn_plan(ctx, fs.plan, (const float *)qp, qs, kc, vc, scale,
                                               fs.general ? fs.mf32 : nullptr, (float *)op, os, s);
            };
        }
        return true;
    }

    // ---- fusions of llama.cpp's layer pattern (the decoder's launch list) ---------------------------
    // A fold: MUL m = RMS_NORM(x) * w read only by MUL_MATs of fewer than 16 tokens: the norm runs inside
    // each of their matvecs (tsr_hip_mul_mat_norm), not as a launch of its own.
    struct Fold {
        int norm = -1, mul = -1;
        const tsr_gg_tensor * x = nullptr;
        const tsr_gg_tensor * w = nullptr;
        float eps = 0.0f;
    };
    // A group: the Q / K / V MUL_MATs (one matvec over their rows concatenated into a plan buffer) with
    // the ROPEs, SET_ROWS and FLASH_ATTN_EXT that read them (one ROPE + SET_ROWS_KV + FA launch for a
    // decode token; ROPE_KV then the planned FA for more tokens); or the gate / up MUL_MATs and their
    // SWIGLU (one matvec with the GLU epilogue over their rows interleaved).
    struct Group {
        bool attn = false;
        int mm_last = -1, fa = -1;
        const tsr_gg_tensor * src1 = nullptr;                  // the MUL_MATs' input
        std::vector<const tsr_gg_tensor *> ws;                 // q, k, v or gate, up
        const tsr_gg_tensor * out = nullptr;                   // GLU: the SWIGLU node
        const tsr_gg_tensor * rq = nullptr;                    // attention: q's ROPE (its parameters)
        const tsr_gg_tensor * kidx = nullptr, * vidx = nullptr;
        uint32_t T = 0;
    };
    std::vector<char> skip;
    std::vector<int> fold_of, group_mm, group_fa;
    std::vector<Fold> folds;
    std::vector<Group> groups;
    std::vector<std::pair<std::vector<uint64_t>, float *>> tables;   // ROPE angle tables of the plan
    std::vector<std::pair<size_t, float *>> rows_bufs;                // Q|K|V row buffers of the plan

    static bool is_(const tsr_gg_tensor * t, int op) { return t != nullptr && t->op == op; }
    bool single(const Graph & g, const tsr_gg_tensor * t) const {   // a node of the graph with one user, not an output
        const int i = g.index_of(t);
        return i >= 0 && g.uses[i] == 1 && !(t->flags & TSR_GG_FLAG_OUTPUT);
    }
    // The weights of MUL_MATs that can share one launch: one device format, one K, in weights buffers.
    bool same_weights(const std::vector<const tsr_gg_tensor *> & mm) const {
        const tsr_gg_tensor * w0 = mm[0]->src[0];
        for (const tsr_gg_tensor * m : mm) {
            const tsr_gg_tensor * w = m->src[0];
            const tsr_gg_tensor * b = w ? base_of(w) : nullptr;
            if (w == nullptr || m->src[1] != mm[0]->src[1] || w->ne[0] != w0->ne[0] || dev_fmt(w->type) != dev_fmt(w0->type) ||
                !loadable(d, w->type) || w->ne[2] != 1 || w->ne[3] != 1 || !contiguous(d, w) || b->buffer == nullptr ||
                b->buffer->usage == TSR_GG_USAGE_COMPUTE || w->view_src != nullptr || m->type != TSR_GG_TYPE_F32)
                return false;
        }
        const int64_t K = w0->ne[0];
        return K >= 32 && K % 32 == 0 && K <= (int64_t)kKMax && (w0->type != TSR_GG_TYPE_Q4_K || K % 256 == 0);
    }

    void find_fusions(const Graph & g) {
        const int n = g.n;
        skip.assign(n, 0);
        fold_of.assign(n, -1);
        group_mm.assign(n, -1);
        group_fa.assign(n, -1);
        // Q / K / V + ROPE + SET_ROWS + FLASH_ATTN_EXT
        for (int i = 0; i < n; ++i) {
            const tsr_gg_tensor * fa = g.nodes[i];
            if (fa->op != TSR_GG_OP_FLASH_ATTN_EXT) continue;
            const tsr_gg_tensor * qp = fa->src[0];
            if (!is_(qp, TSR_GG_OP_PERMUTE) || qp->op_params[0] != 0 || qp->op_params[1] != 2 || qp->op_params[2] != 1 ||
                !single(g, qp))
                continue;
            const tsr_gg_tensor * rq = qp->src[0];
            if (!is_(rq, TSR_GG_OP_ROPE) || !single(g, rq) || rq->src[2] != nullptr) continue;
            const tsr_gg_tensor * shq = rq->src[0];
            if (!is_(shq, TSR_GG_OP_RESHAPE) || !single(g, shq) || !is_(shq->src[0], TSR_GG_OP_MUL_MAT) || !single(g, shq->src[0]))
                continue;
            const tsr_gg_tensor * mq = shq->src[0];
            const tsr_gg_tensor * srk = nullptr, * srv = nullptr;
            for (int j = 0; j < i; ++j) {
                const tsr_gg_tensor * t = g.nodes[j];
                if (t->op != TSR_GG_OP_SET_ROWS) continue;
                if (base_of(t)->data == base_of(fa->src[1])->data) srk = t;
                if (base_of(t)->data == base_of(fa->src[2])->data) srv = t;
            }
            if (srk == nullptr || srv == nullptr || g.uses[g.index_of(srk)] || g.uses[g.index_of(srv)]) continue;
            // K: SET_ROWS(cache_k, VIEW(ROPE(RESHAPE(MUL_MAT)))), V: SET_ROWS(cache_v, VIEW(RESHAPE(MUL_MAT)))
            const tsr_gg_tensor * vk = srk->src[0], * vv = srv->src[0];
            if (!is_(vk, TSR_GG_OP_VIEW) || !single(g, vk) || !is_(vv, TSR_GG_OP_VIEW) || !single(g, vv)) continue;
            const tsr_gg_tensor * rk = vk->src[0], * shv = vv->src[0];
            if (!is_(rk, TSR_GG_OP_ROPE) || !single(g, rk) || rk->src[1] != rq->src[1] || rk->src[2] != nullptr) continue;
            if (memcmp(rk->op_params + 1, rq->op_params + 1, 15 * 4) != 0) continue;
            const tsr_gg_tensor * shk = rk->src[0];
            if (!is_(shk, TSR_GG_OP_RESHAPE) || !single(g, shk) || !is_(shk->src[0], TSR_GG_OP_MUL_MAT) || !single(g, shk->src[0]))
                continue;
            if (!is_(shv, TSR_GG_OP_RESHAPE) || !single(g, shv) || !is_(shv->src[0], TSR_GG_OP_MUL_MAT) || !single(g, shv->src[0]))
                continue;
            const tsr_gg_tensor * mk = shk->src[0], * mv = shv->src[0];
            if (!same_weights({mq, mk, mv})) continue;
            const uint32_t D = (uint32_t)rq->ne[0], H = (uint32_t)rq->ne[1], T = (uint32_t)rq->ne[2];
            const uint32_t Hk = (uint32_t)rk->ne[1], E = Hk * D;
            const int32_t n_dims = rq->op_params[1], mode = rq->op_params[2];
            if (mq->ne[0] != (int64_t)H * D || mk->ne[0] != E || mv->ne[0] != E || nrows(mq) != T || nrows(mk) != T ||
                nrows(mv) != T || rk->ne[0] != D || rk->ne[2] != T || vk->ne[0] != E || vv->ne[0] != E || vk->ne[1] != T ||
                vv->ne[1] != T || vk->nb[1] != 4ull * E || vv->nb[1] != 4ull * E || !same_shape(rq, shq) || !same_shape(rk, shk))
                continue;
            if (mode != TSR_HIP_ROPE_NORMAL && mode != TSR_HIP_ROPE_NEOX && mode != TSR_HIP_ROPE_IMROPE) continue;
            if (param_f32(rq, 6) != 1.0f || param_f32(rq, 7) != 0.0f || rq->op_params[15] != 0 || n_dims < 2 || n_dims % 2 ||
                (uint32_t)n_dims > D)
                continue;
            const uint32_t G = Hk ? H / Hk : 0;
            const uint32_t row = H * D + 2 * E;
            if (Hk == 0 || H % Hk || D % 32 || row > 16384) continue;
            if (T == 1 && ((D != 64 && D != 128) || (G + 2) * D > 1024 || n_dims % 8 || (uint32_t)n_dims > std::min(D, 128u)))
                continue;
            const tsr_gg_tensor * kidx = srk->src[1], * vidx = srv->src[1];
            if (kidx == nullptr || vidx == nullptr || kidx->type != TSR_GG_TYPE_I64 || vidx->type != TSR_GG_TYPE_I64 ||
                kidx->ne[0] != T || vidx->ne[0] != T || kidx->op != TSR_GG_OP_NONE || vidx->op != TSR_GG_OP_NONE ||
                g.index_of(kidx) >= 0 || g.index_of(vidx) >= 0)
                continue;
            const tsr_gg_tensor * pos = rq->src[1];
            if (pos == nullptr || pos->type != TSR_GG_TYPE_I32) continue;
            Group gr;
            gr.attn = true;
            gr.fa = i;
            gr.mm_last = std::max({g.index_of(mq), g.index_of(mk), g.index_of(mv)});
            gr.src1 = mq->src[1];
            gr.ws = {mq->src[0], mk->src[0], mv->src[0]};
            gr.rq = rq;
            gr.kidx = kidx;
            gr.vidx = vidx;
            gr.T = T;
            // the input must be intact when the fused matvec reads it, at the last of the three
            const int first = std::min({g.index_of(mq), g.index_of(mk), g.index_of(mv)});
            if (g.written_between(first, gr.mm_last, gr.src1->data, gr.src1->data + nbytes_of(d, gr.src1))) continue;
            groups.push_back(gr);
            const int gi = (int)groups.size() - 1;
            group_mm[gr.mm_last] = gi;
            group_fa[i] = gi;
            for (const tsr_gg_tensor * t : {mq, mk, mv, shq, shk, shv, rq, rk, vk, vv, srk, srv, qp}) skip[g.index_of(t)] = 1;
        }
        // gate / up + SWIGLU
        for (int i = 0; i < n; ++i) {
            const tsr_gg_tensor * u = g.nodes[i];
            if (u->op != TSR_GG_OP_GLU || u->op_params[0] != TSR_GG_GLU_SWIGLU || u->op_params[1] != 0 || u->src[1] == nullptr)
                continue;
            const tsr_gg_tensor * mg = u->src[0], * mu = u->src[1];
            if (!is_(mg, TSR_GG_OP_MUL_MAT) || !is_(mu, TSR_GG_OP_MUL_MAT) || !single(g, mg) || !single(g, mu) || mg == mu ||
                !same_weights({mg, mu}) || mg->src[0]->ne[1] != mu->src[0]->ne[1] || !same_shape(u, mg) ||
                !same_shape(mg, mu) || u->type != TSR_GG_TYPE_F32)
                continue;
            const uint32_t T = (uint32_t)nrows(mg);
            if (dev_fmt(mg->src[0]->type) == TSR_HIP_FMT_Q8_0 && T >= 16) continue;   // GLU: Q8_0 on the matvec kernels only
            const int a = g.index_of(mg), b = g.index_of(mu);
            const tsr_gg_tensor * x = mg->src[1];
            const uint64_t xl = x->data, xh = x->data + nbytes_of(d, x);
            const uint64_t ul = u->data, uh = u->data + nbytes_of(d, u);
            if (g.written_between(std::min(a, b), i, xl, xh) || (ul < xh && xl < uh)) continue;
            Group gr;
            gr.mm_last = i;
            gr.src1 = x;
            gr.ws = {mg->src[0], mu->src[0]};
            gr.out = u;
            gr.T = T;
            groups.push_back(gr);
            group_mm[i] = (int)groups.size() - 1;
            skip[a] = skip[b] = 1;
        }
        // RMS_NORM * w folded into the MUL_MATs (and groups) that read it
        for (int m = 0; m < n; ++m) {
            const tsr_gg_tensor * mt = g.nodes[m];
            if (mt->op != TSR_GG_OP_MUL || mt->type != TSR_GG_TYPE_F32 || (mt->flags & TSR_GG_FLAG_OUTPUT) || g.users[m].empty())
                continue;
            const tsr_gg_tensor * nt = is_(mt->src[0], TSR_GG_OP_RMS_NORM) ? mt->src[0] : mt->src[1];
            const tsr_gg_tensor * w = nt == mt->src[0] ? mt->src[1] : mt->src[0];
            if (!is_(nt, TSR_GG_OP_RMS_NORM) || !single(g, nt) || w == nullptr || w->type != TSR_GG_TYPE_F32 ||
                w->ne[0] != mt->ne[0] || nrows(w) != 1 || !contiguous(d, w) || !same_shape(nt, mt))
                continue;
            const tsr_gg_tensor * x = nt->src[0];
            const int64_t K = mt->ne[0], T = nrows(mt);
            if (x == nullptr || !same_shape(x, nt) || K > 8192 || T >= 16 || mt->ne[2] != 1 || mt->ne[3] != 1) continue;
            bool ok = true;
            int last = m;
            for (int u : g.users[m]) {
                const tsr_gg_tensor * ut = g.nodes[u];
                // a reader: a MUL_MAT of m (alone, or in a group), not one whose result gets an epilogue
                ok &= ut->op == TSR_GG_OP_MUL_MAT && ut->src[1] == mt && ut->src[0] != mt;
                const int nx = g.next_real(u);
                ok &= !(nx >= 0 && g.nodes[nx]->op == TSR_GG_OP_SCALE && g.only_user(u, nx));
                const int gm = ok ? (skip[u] ? -1 : u) : -1;
                (void)gm;
                last = std::max(last, u);
            }
            for (const Group & gr : groups) if (gr.src1 == mt) last = std::max(last, gr.mm_last);
            const int ni = g.index_of(nt);
            if (!ok || ni < 0 || g.written_between(ni, last + 1, x->data, x->data + nbytes_of(d, x))) continue;
            Fold f;
            f.norm = ni;
            f.mul = m;
            f.x = x;
            f.w = w;
            f.eps = param_f32(nt, 0);
            folds.push_back(f);
            fold_of[m] = (int)folds.size() - 1;
            skip[ni] = skip[m] = 1;
        }
    }

    // A device buffer owned by the plan (build mode).
    void * plan_buf(size_t bytes) {
        void * p = nullptr;
        if (tsr_hip_alloc(d->ctx, bytes, &p) != TSR_HIP_OK) return nullptr;
        plan->bufs.push_back(p);
        return p;
    }

    // The matvec of a group (or of a MUL_MAT with a folded norm): y = W x (the norm applied to x first).
    bool group_matvec(const Graph & g, const Group & gr, int at) {
        const tsr_gg_tensor * x = gr.src1;
        const int fi = g.index_of(x) >= 0 ? fold_of[g.index_of(x)] : -1;
        const Fold * fo = fi >= 0 ? &folds[fi] : nullptr;
        Rows X, Y, NW;
        if (!f32_rows(d, fo ? fo->x : x, "src1", &X, &why)) return false;
        if (fo && !f32_rows(d, fo->w, "norm weight", &NW, &why)) return false;
        Weight * wt = nullptr;
        const int rc = fused_weight_of(d, gr.ws, !gr.attn, build, &wt, &why);
        if (rc) {
            if (rc != TSR_GG_E_UNSUPPORTED) why = d->err;
            return false;
        }
        const uint32_t T = X.rows, N = wt->N, K = wt->K;
        uint32_t flags = 0;
        uint64_t ys;
        if (gr.attn) {
            ys = N;
            Y.a = 0;
            if (build) {
                Y.p = nullptr;
                for (auto & rb : rows_bufs)
                    if (rb.first >= (size_t)T * N * 4) Y.p = rb.second;
                if (Y.p == nullptr) {
                    Y.p = plan_buf((size_t)T * N * 4);
                    if (Y.p == nullptr) return refuse("no device memory for the Q|K|V rows");
                    rows_bufs.emplace_back((size_t)T * N * 4, (float *)Y.p);
                }
            }
        } else {
            if (!f32_rows(d, gr.out, "SWIGLU result", &Y, &why)) return false;
            ys = Y.stride;
            flags = TSR_HIP_MM_GLU;
        }
        Call & c = add(TSR_GG_CALL_MUL_MAT, at);
        c.info.N = N;
        c.info.K = K;
        c.info.T = T;
        c.info.flags = flags;
        c.info.x = X.a;
        c.info.y = Y.a;
        c.info.w = gr.ws[0]->data;
        c.info.x_stride = X.stride;
        c.info.y_stride = ys;
        c.info.node2 = fo ? fo->norm : -1;
        c.info.scale = fo ? fo->eps : 0.0f;
        c.info.add = fo ? NW.a : 0;
        c.capturable = T < 16;
        if (build) {
            tsr_hip_ctx * ctx = d->ctx;
            const tsr_hip_weight * hw = wt->w;
            const float * xp = (const float *)X.p;
            float * yp = (float *)Y.p;
            const uint64_t xs = X.stride;
            void * s = stream();
            if (fo) {
                const float eps = fo->eps;
                const float * nw = (const float *)NW.p;
                c.run = [=](const Plan &) { return tsr_hip_mul_mat_norm(ctx, hw, xp, T, xs, eps, nw, yp, ys, nullptr, 0, flags, s); };
                if (gr.attn && T == 1u && fuse) qkv_in = QkvIn{ (int)plan->calls.size() - 1, hw, xp, nw, eps };
            } else {
                c.run = [=](const Plan &) { return tsr_hip_mul_mat(ctx, hw, xp, T, xs, yp, ys, nullptr, 0, flags, s); };
            }
            if (gr.attn) qkv_rows = yp;
        } else if (fo && gr.attn && T == 1u && fuse) {
            qkv_in = QkvIn{ (int)plan->calls.size() - 1, nullptr, nullptr, nullptr, 0.0f };
        }
        if (qkv_in.call >= 0) {                            // what the attention call will read, and where
            span(X, &qkv_in.x_lo, &qkv_in.x_hi);
            span(NW, &qkv_in.w_lo, &qkv_in.w_hi);
        }
        return true;
    }
    float * qkv_rows = nullptr;                            // the Q|K|V rows of the group being emitted
    // A one-token Q|K|V MUL_MAT with its norm folded in: the attention call of its group runs it
    // (tsr_hip_attn_qkv_plan_rope_tab) and its own call becomes a no-op marked TSR_GG_CALL_IN_NEXT.
    struct QkvIn {
        int call = -1;
        const tsr_hip_weight * w = nullptr;
        const float * x = nullptr;
        const float * nw = nullptr;
        float eps = 0.0f;
        uint64_t x_lo = 0, x_hi = 0, w_lo = 0, w_hi = 0;   // ggml bytes of x and of the norm weight
    };
    QkvIn qkv_in;                                          // of the group being emitted

    // The attention of a group: ROPE of q and k, SET_ROWS of k and v, FLASH_ATTN_EXT.
    bool group_attn(const Graph & g, const Group & gr) {
        FaInfo f;
        if (!fa_info(g, gr.fa, &f)) return false;
        const tsr_gg_tensor * rq = gr.rq;
        RopeFacts rf;                                          // the q rotation the call performs
        if (!rope_rules(rq, &rf)) return false;
        const int32_t n_dims = rf.n_dims, mode = rf.mode;
        const float base = rf.base, attn = param_f32(rq, 8);
        const tsr_gg_tensor * pos = rf.pos;
        void *pp = nullptr, *kp = nullptr;
        std::string w2;
        if (!dev_ptr(d, pos->data, 4 * (size_t)pos->ne[0], &pp, &w2) || !dev_ptr(d, gr.kidx->data, 8 * (size_t)gr.T, &kp, &w2))
            return refuse("attention device-inputs: positions and cell indices in device memory of this device (%s)",
                          w2.c_str());
        const uint32_t T = gr.T, row = f.H * f.D + 2 * f.Hk * f.D;
        float * tab = nullptr;
        if (T == 1) {                                        // the token's angle table, once per graph
            const std::vector<uint64_t> key{pos->data, (uint64_t)(uint32_t)n_dims, (uint64_t)(uint32_t)rq->op_params[5],
                                            (uint64_t)(uint32_t)rq->op_params[8]};
            for (auto & t : tables) if (t.first == key) tab = t.second;
            if (tab == nullptr) {
                Call & tc = add(TSR_GG_CALL_ROPE_TABLE, gr.fa);
                tc.info.x = pos->data;
                tc.info.n_dims = (uint32_t)n_dims;
                tc.info.scale = base;
                tc.info.scale2 = attn;
                if (build) {
                    tab = (float *)plan_buf(4 * (size_t)n_dims + 64);
                    if (tab == nullptr) return refuse("no device memory for the ROPE table");
                    tsr_hip_ctx * ctx = d->ctx;
                    void * s = stream();
                    float * tb = tab;
                    const uint32_t nd = (uint32_t)n_dims;
                    tc.run = [=](const Plan &) { return tsr_hip_rope_table(ctx, (const int32_t *)pp, nd, base, attn, tb, s); };
                } else {
                    tab = (float *)(uintptr_t)(0x1000 + 64 * tables.size());     // describe mode: a marker
                }
                tables.emplace_back(key, tab);
            }
        } else {
            Call & rc = add(TSR_GG_CALL_ROPE_KV, gr.fa);
            rc.info.T = T;
            rc.info.x_stride = row;
            rc.info.n_dims = (uint32_t)n_dims;
            rc.info.mode = (uint32_t)mode;
            rc.info.scale = base;
            rc.info.add = gr.kidx->data;
        }
        // the one-token Q|K|V MUL_MAT moves into this call only while its x and norm weight still hold at
        // this node what they held at the MUL_MATs' place (no node in between writes them: ggml-alloc may
        // give bytes whose last reader has run to a later node)
        if (qkv_in.call >= 0 && (g.written_between(gr.mm_last, gr.fa, qkv_in.x_lo, qkv_in.x_hi) ||
                                 g.written_between(gr.mm_last, gr.fa, qkv_in.w_lo, qkv_in.w_hi)))
            qkv_in = QkvIn{};
        Call & c = add(TSR_GG_CALL_FLASH_ATTN, gr.fa);
        fa_call_info(c, f, 0, row, g.nodes[gr.fa]->data);
        if (T == 1 && qkv_in.call >= 0) plan->calls[qkv_in.call].info.flags |= TSR_GG_CALL_IN_NEXT;
        c.info.n_dims = (uint32_t)n_dims;
        c.info.mode = (uint32_t)mode;
        c.info.node2 = gr.mm_last;
        if (build) {
            uint32_t cell, bir;
            const KvTensor * kt = kv_at(d, f.kbase, &cell, &bir);
            const KvTensor * vt = kv_at(d, f.vbase, &cell, &bir);
            if (kt == nullptr || vt == nullptr) return refuse("FLASH_ATTN_EXT: the KV caches are not placed");
            if (f.kidx != gr.kidx->data) return refuse("attention: the new cells are not the K SET_ROWS' indices");
            const int slot = fa_slot(f, gr.vidx->data);
            if (slot < 0) return false;
            tsr_hip_ctx * ctx = d->ctx;
            tsr_hip_kv * kc = kt->kv;
            tsr_hip_kv * vc = vt->kv;
            void * s = stream();
            void * op = f.op;
            const uint64_t os = f.os;
            const float scale = f.scale;
            float * qkv = qkv_rows;
            const uint32_t nd = (uint32_t)n_dims, D = f.D, H = f.H, Hk = f.Hk;
            const int64_t * cells = (const int64_t *)kp;
            if (T == 1 && qkv_in.call >= 0) {                // the group's Q|K|V MUL_MAT runs here
                const float * tb = tab;
                const QkvIn q = qkv_in;
                plan->calls[q.call].run = [](const Plan &) { return (int)TSR_HIP_OK; };
                c.run = [=](const Plan & pl) {
                    const FaSlot & fs = pl.fa[slot];
                    return tsr_hip_attn_qkv_plan_rope_tab(ctx, fs.plan, q.w, q.x, q.eps, q.nw, qkv, kc, vc, scale, nd, mode,
                                                          tb, cells, nullptr, fs.general ? fs.mf32 : nullptr, (float *)op,
                                                          os, s);
                };
            } else if (T == 1) {
                const float * tb = tab;
                c.run = [=](const Plan & pl) {
                    const FaSlot & fs = pl.fa[slot];
                    return tsr_hip_flash_attn_plan_rope_tab(ctx, fs.plan, qkv, kc, vc, scale, nd, mode, tb, cells, nullptr,
                                                            fs.general ? fs.mf32 : nullptr, (float *)op, os, s);
                };
            } else {
                Call & rc = plan->calls[plan->calls.size() - 2];
                const int32_t * pv = (const int32_t *)pp;
                rc.run = [=](const Plan &) {
                    return tsr_hip_rope_kv(ctx, qkv, T, row, D, H, Hk, nd, mode, pv, base, attn, kc, vc, cells, nullptr, s);
                };
                c.run = [=](const Plan & pl) {
                    const FaSlot & fs = pl.fa[slot];
                    return tsr_hip_flash_attn_plan(ctx, fs.plan, qkv, row, kc, vc, scale, fs.general ? fs.mf32 : nullptr,
                                                   (float *)op, os, s);
                };
            }
        }
        return true;
    }

    // Every node of the graph in order; the nodes a call absorbed are skipped.
    bool lower(const Graph & g, int * bad_node) {
        fuse = (d->options & TSR_GG_OPT_NO_FUSION) == 0u;
        if (fuse) find_fusions(g);
        else {
            skip.assign(g.n, 0);
            fold_of.assign(g.n, -1);
            group_mm.assign(g.n, -1);
            group_fa.assign(g.n, -1);
        }
        for (int i = 0; i < g.n; ++i) {
            const tsr_gg_tensor * node = g.nodes[i];
            if (group_mm[i] >= 0) {
                const Group & gr = groups[group_mm[i]];
                if (!group_matvec(g, gr, i)) {
                    *bad_node = i;
                    return false;
                }
                if (gr.attn) {
                    pending_qkv[group_mm[i]] = qkv_rows;
                    pending_in[group_mm[i]] = qkv_in;
                    qkv_in = QkvIn{};
                }
                if (!gr.attn) continue;                        // the SWIGLU node is this call
            }
            if (group_fa[i] >= 0) {
                qkv_rows = pending_qkv[group_fa[i]];
                qkv_in = pending_in.count(group_fa[i]) ? pending_in[group_fa[i]] : QkvIn{};
                if (!group_attn(g, groups[group_fa[i]])) {
                    *bad_node = i;
                    return false;
                }
                continue;
            }
            if (is_noop(node->op) || skip[i]) continue;
            int consumed = i;
            bool ok;
            switch (node->op) {
                case TSR_GG_OP_MUL_MAT: ok = mul_mat(g, i, &consumed); break;
                case TSR_GG_OP_RMS_NORM: ok = rms_norm(g, i, &consumed); break;
                case TSR_GG_OP_ADD: ok = add_op(g, i); break;
                case TSR_GG_OP_ROPE: ok = rope(g, i); break;
                case TSR_GG_OP_GLU: ok = glu(g, i); break;
                case TSR_GG_OP_GET_ROWS: ok = get_rows(g, i); break;
                case TSR_GG_OP_ARGMAX: ok = argmax(g, i); break;
                case TSR_GG_OP_SET_ROWS: ok = set_rows(g, i); break;
                case TSR_GG_OP_FLASH_ATTN_EXT: ok = flash_attn(g, i); break;
                case TSR_GG_OP_MUL:
                    ok = refuse("MUL norm-weight: the weight multiply right behind an RMS_NORM it alone reads [%s]",
                                dims(node).c_str());
                    break;
                case TSR_GG_OP_SCALE:
                case TSR_GG_OP_UNARY:
                    ok = refuse("SCALE/TANH epilogue: only as the tail of a MUL_MAT it alone reads [%s]", dims(node).c_str());
                    break;
                default: ok = refuse("op %d: not on the device (no kernel for it)", node->op); break;
            }
            if (!ok) {
                *bad_node = i;
                return false;
            }
            // the nodes between i and the last fused one are no-ops (next_real): skip to it
            i = consumed;
        }
        for (const Call & c : plan->calls) plan->capturable &= c.capturable;
        return true;
    }
    std::map<int, float *> pending_qkv;                     // group -> its Q|K|V rows (between the two emissions)
    std::map<int, QkvIn> pending_in;                        // group -> its one-token Q|K|V MUL_MAT (to run inside)
};

Graph make_graph(const tsr_gg_dev * d, const tsr_gg_tensor * const * nodes, int n) {
    Graph g{nodes, n, std::vector<int>(n, 0), std::vector<std::vector<int>>(n), {}};
    std::map<const tsr_gg_tensor *, int> at;
    for (int i = 0; i < n; ++i) at.emplace(nodes[i], i);
    for (int j = 0; j < n; ++j) {
        for (int s = 0; s < 10; ++s) {
            auto it = nodes[j]->src[s] ? at.find(nodes[j]->src[s]) : at.end();
            if (it != at.end() && it->second < j) {
                ++g.uses[it->second];
                g.users[it->second].push_back(j);
            }
        }
        // (a view names its parent in src[0]: a chain of views is a chain of uses)
    }
    g.out.resize(n);
    for (int i = 0; i < n; ++i) {
        const tsr_gg_tensor * t = nodes[i];
        if (is_noop(t->op)) continue;
        const tsr_gg_tensor * b = t->op == TSR_GG_OP_SET_ROWS ? base_of(t) : t;
        g.out[i] = {b->data, b->data + nbytes_of(d, b)};
    }
    return g;
}

// The FLASH_ATTN_EXT chunk lists of a plan from the masks and new cells of this run.
int refresh_fa(tsr_gg_dev * d, Plan & p, bool * changed) {
    *changed = false;
    for (FaSlot & f : p.fa) {
        std::vector<uint32_t> words;
        const Mask * m = nullptr;
        if (f.mask) {
            auto it = d->masks.find(f.mask);
            if (it == d->masks.end())
                return d->fail(TSR_GG_E_UNSUPPORTED, "FLASH_ATTN_EXT: its mask was not written by the host (no summary)");
            m = &it->second;
            if (m->n_q != f.T || m->n_kv != f.n_kv)
                return d->fail(TSR_GG_E_UNSUPPORTED, "FLASH_ATTN_EXT: the mask summary is %u x %u, the op %u x %u", m->n_q, m->n_kv,
                               f.T, f.n_kv);
            words = m->words;
        } else {                                        // no mask: every cell visible
            words.assign(8 + 4 * (size_t)f.T, 0u);
            words[0] = 0x4D55534Du;
            words[1] = f.T;
            words[2] = f.n_kv;
            for (uint32_t q = 0; q < f.T; ++q) words[8 + 4 * q + 1] = f.n_kv;
        }
        std::vector<uint32_t> runs;                     // runs of consecutive new cells
        if (f.kidx) {
            auto it = d->shadows.find(f.kidx);
            if (it == d->shadows.end() || it->second.size() < 8 * (size_t)f.kidx_n)
                return d->fail(TSR_GG_E_UNSUPPORTED, "FLASH_ATTN_EXT: the new-cell indices were not written by the host");
            if (f.vidx) {                                   // one launch stores k and v into the K indices' cells
                auto iv = d->shadows.find(f.vidx);
                if (iv == d->shadows.end() || iv->second.size() < 8 * (size_t)f.kidx_n ||
                    memcmp(iv->second.data(), it->second.data(), 8 * (size_t)f.kidx_n) != 0)
                    return d->fail(TSR_GG_E_UNSUPPORTED, "attention: the K and V SET_ROWS write different cells");
            }
            const int64_t * ix = (const int64_t *)it->second.data();
            for (uint32_t j = 0; j < f.kidx_n; ++j) {
                if (ix[j] < 0 || ix[j] > 0xFFFFFFFFll) return d->fail(TSR_GG_E_ARG, "FLASH_ATTN_EXT: new cell %lld", (long long)ix[j]);
                const uint32_t c = (uint32_t)ix[j];
                if (!runs.empty() && runs.back() == c) runs.back() = c + 1;
                else { runs.push_back(c); runs.push_back(c + 1); }
            }
        }
        f.general = (words[3] & 1u) != 0;
        if (f.general) {
            if (f.mf32 == nullptr) {
                void * pm = nullptr;
                const int rc = tsr_hip_alloc(d->ctx, f.mf32_floats * 4, &pm);
                if (rc) return d->hip(rc, "FA mask copy");
                f.mf32 = (float *)pm;
            }
            std::vector<float> mf(f.mf32_floats);
            int rc = tsr_hip_msum_mask_f32(m->f16.data(), m->n_kv, m->n_kv, m->n_q, f.scale, mf.data());
            if (rc == 0) rc = tsr_hip_write(d->ctx, f.mf32, mf.data(), mf.size() * 4);
            if (rc) return d->hip(rc, "FA mask copy");
        }
        int ch = 0;
        const int rc = tsr_hip_fa_plan_set(d->ctx, f.plan, words.data(), f.general ? 1 : 0,
                                           runs.empty() ? nullptr : (const uint32_t (*)[2])runs.data(),
                                           (uint32_t)(runs.size() / 2), &ch, d->stream);
        if (rc) return d->hip(rc, "FA plan");
        *changed |= ch != 0;
    }
    return TSR_GG_OK;
}

int run_calls(tsr_gg_dev * d, Plan & p, const tsr_gg_tensor * const * nodes) {
    for (Call & c : p.calls) {
        const int rc = c.run(p);
        if (rc) return d->fail(rc == TSR_HIP_E_NOMEM ? TSR_GG_E_NOMEM : TSR_GG_E_DEVICE, "node '%s': %s",
                               nodes ? nodes[c.info.node]->name : "?", tsr_hip_strerror(rc));
    }
    return TSR_GG_OK;
}

int capture(tsr_gg_dev * d, Plan & p) {
    if (p.graph) tsr_hip_graph_free(d->ctx, p.graph);
    p.graph = nullptr;
    int rc = tsr_hip_graph_begin(d->ctx, d->stream);
    if (rc) return d->hip(rc, "graph capture");
    const int rr = run_calls(d, p, nullptr);
    tsr_hip_graph * gr = nullptr;
    rc = tsr_hip_graph_end(d->ctx, d->stream, &gr);
    if (rr) {
        if (gr) tsr_hip_graph_free(d->ctx, gr);
        return rr;
    }
    if (rc) return d->hip(rc, "graph capture");
    p.graph = gr;
    d->st.captures++;
    return TSR_GG_OK;
}

}  // namespace

// ---------------------------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------------------------
extern "C" {

int tsr_gg_open(int device, tsr_gg_dev ** out) {
    if (out == nullptr || device < -1) return TSR_GG_E_ARG;
    *out = nullptr;
    auto * d = new (std::nothrow) tsr_gg_dev();
    if (d == nullptr) return TSR_GG_E_NOMEM;
    d->device = device;
    if (device >= 0) {
        const int rc = tsr_hip_open(device, &d->ctx);
        if (rc) {
            delete d;
            return rc == TSR_HIP_E_NODEV ? TSR_GG_E_NODEV : TSR_GG_E_DEVICE;
        }
        d->stream = tsr_hip_stream(d->ctx);
    }
    *out = d;
    return TSR_GG_OK;
}

int tsr_gg_close(tsr_gg_dev * d) {
    if (d == nullptr) return TSR_GG_E_ARG;
    {
        std::lock_guard<std::recursive_mutex> lk(d->mtx);
        drop_plans(d);
        for (auto & [a, w] : d->weights) if (d->ctx && w.w) tsr_hip_weight_free(d->ctx, w.w);
        for (auto & [a, w] : d->fused) if (d->ctx && w.w) tsr_hip_weight_free(d->ctx, w.w);
        d->weights.clear();
        d->fused.clear();
        while (!d->buffers.empty()) tsr_gg_buffer_free(d->buffers.back());
        if (d->ctx) tsr_hip_close(d->ctx);
        d->ctx = nullptr;
    }
    delete d;
    return TSR_GG_OK;
}

const char * tsr_gg_last_error(const tsr_gg_dev * d) { return d ? d->err.c_str() : "no device"; }
void * tsr_gg_hip_ctx(tsr_gg_dev * d) { return d ? (void *)d->ctx : nullptr; }

int tsr_gg_register_type(tsr_gg_dev * d, const char * name, uint32_t blck_size, uint32_t type_size, tsr_gg_to_float_fn to_float,
                         int32_t * id) {
    if (d == nullptr || id == nullptr || to_float == nullptr || blck_size == 0 || type_size == 0 || blck_size % 32 != 0)
        return TSR_GG_E_ARG;
    std::lock_guard<std::recursive_mutex> lk(d->mtx);
    if (d->foreign.size() >= 64) return TSR_GG_E_ARG;
    d->foreign.push_back({blck_size, type_size, to_float, name ? name : "foreign"});
    *id = TSR_GG_TYPE_FOREIGN + (int32_t)d->foreign.size() - 1;
    return TSR_GG_OK;
}

size_t tsr_gg_alignment(void) { return kAlign; }

size_t tsr_gg_alloc_size(const tsr_gg_dev * d, const tsr_gg_tensor * t) {
    if (t == nullptr) return 0;
    const size_t n = nbytes_of(d, t);
    return (n + kAlign - 1) / kAlign * kAlign;
}

int tsr_gg_buffer_alloc(tsr_gg_dev * d, size_t size, int usage, tsr_gg_buffer ** out) {
    if (d == nullptr || out == nullptr || size >= kVSpan) return TSR_GG_E_ARG;
    std::lock_guard<std::recursive_mutex> lk(d->mtx);
    auto * b = new (std::nothrow) tsr_gg_buffer();
    if (b == nullptr) return TSR_GG_E_NOMEM;
    b->dev = d;
    b->vbase = d->next_vbase;
    d->next_vbase += kVSpan;
    b->size = (size + kAlign - 1) / kAlign * kAlign;
    b->usage = usage;
    d->buffers.push_back(b);
    *out = b;
    return TSR_GG_OK;
}

int tsr_gg_buffer_set_usage(tsr_gg_buffer * b, int usage) {
    if (b == nullptr) return TSR_GG_E_ARG;
    std::lock_guard<std::recursive_mutex> lk(b->dev->mtx);
    if (b->mode != kUndecided && (usage == TSR_GG_USAGE_WEIGHTS) != (b->mode == kWeights) && b->mode != kKv)
        b->mode = usage == TSR_GG_USAGE_WEIGHTS ? kWeights : kLinear;
    b->usage = usage;
    return TSR_GG_OK;
}

uint64_t tsr_gg_buffer_base(const tsr_gg_buffer * b) { return b ? b->vbase : 0; }
size_t tsr_gg_buffer_size(const tsr_gg_buffer * b) { return b ? b->size : 0; }
int tsr_gg_buffer_mode(const tsr_gg_buffer * b) { return b ? b->mode : -1; }

int tsr_gg_buffer_init_tensor(tsr_gg_buffer * b, const tsr_gg_tensor * t) {
    if (b == nullptr || t == nullptr) return TSR_GG_E_ARG;
    tsr_gg_dev * d = b->dev;
    std::lock_guard<std::recursive_mutex> lk(d->mtx);
    if (t->view_src != nullptr) return TSR_GG_OK;                // views add nothing
    const size_t n = nbytes_of(d, t);
    if (t->data < b->vbase || t->data + n > b->vbase + b->size)
        return d->fail(TSR_GG_E_ARG, "init_tensor: '%s' lies outside its buffer", t->name);
    if (b->mode != kUndecided)
        return TSR_GG_OK;                                          // late tensors keep the decided storage
    TInfo ti;
    ti.name = t->name;
    ti.vaddr = t->data;
    ti.nbytes = n;
    ti.type = t->type;
    memcpy(ti.ne, t->ne, sizeof ti.ne);
    memcpy(ti.nb, t->nb, sizeof ti.nb);
    b->tensors.push_back(ti);
    return TSR_GG_OK;
}

static int buf_enter(tsr_gg_buffer * b, const tsr_gg_tensor * t, size_t offset, size_t size, uint64_t * addr) {
    tsr_gg_dev * d = b->dev;
    if (d->ctx == nullptr) return d->fail(TSR_GG_E_NODEV, "a probe device has no memory");
    const int rc = decide(d, b);
    if (rc) return rc;
    const uint64_t a = t ? t->data + offset : b->vbase + offset;
    if (a < b->vbase || a + size > b->vbase + b->size)
        return d->fail(TSR_GG_E_ARG, "bytes [0x%llx, +%zu) outside the buffer", (unsigned long long)a, size);
    *addr = a;
    return TSR_GG_OK;
}

int tsr_gg_buffer_set_tensor(tsr_gg_buffer * b, const tsr_gg_tensor * t, const void * data, size_t offset, size_t size) {
    if (b == nullptr || t == nullptr || (size && data == nullptr)) return TSR_GG_E_ARG;
    tsr_gg_dev * d = b->dev;
    std::lock_guard<std::recursive_mutex> lk(d->mtx);
    uint64_t a;
    int rc = buf_enter(b, t, offset, size, &a);
    if (rc || size == 0) return rc;
    if (b->mode == kKv) return kv_access(d, b, a, size, (const uint8_t *)data, nullptr, 0);
    drop_weights_in(d, a, a + size);
    // stream-ordered: small inputs through the library's pinned staging, the rest synchronously
    rc = size <= 16384 ? tsr_hip_write_async(d->ctx, b->mem + (a - b->vbase), data, size, d->stream)
                       : tsr_hip_write(d->ctx, b->mem + (a - b->vbase), data, size);
    if (rc) return d->hip(rc, t->name);
    // host copies: index inputs (new-cell runs) and KQ masks (their summaries)
    const uint64_t t0 = t->data;
    const size_t tn = nbytes_of(d, t);
    if ((t->type == TSR_GG_TYPE_I64 || t->type == TSR_GG_TYPE_I32) && tn <= kShadowMax) {
        std::vector<uint8_t> & sh = d->shadows[t0];
        sh.resize(tn);
        memcpy(sh.data() + offset, data, std::min(size, tn - offset));
    }
    if (t->type == TSR_GG_TYPE_F16 && strstr(t->name, "kq_mask") != nullptr && t->ne[2] == 1 && t->ne[3] == 1 &&
        t->ne[0] >= 1 && t->ne[1] >= 1 && t->nb[0] == 2) {
        Mask & m = d->masks[t0];
        const uint32_t n_kv = (uint32_t)t->ne[0], n_q = (uint32_t)t->ne[1];
        const size_t rs = t->nb[1] / 2;
        if (m.n_kv != n_kv || m.n_q != n_q) {
            m = Mask{};
            m.n_kv = n_kv;
            m.n_q = n_q;
            m.f16.assign((size_t)n_kv * n_q, 0xFC00u);
        }
        // the written bytes into the dense host copy (rows of n_kv)
        const uint8_t * src = (const uint8_t *)data;
        for (size_t o = 0; o < size; o += 2) {
            const size_t e = (offset + o) / 2, r = e / rs, c = e % rs;
            if (r < n_q && c < n_kv) memcpy(&m.f16[r * n_kv + c], src + o, 2);
        }
        m.words.assign(8 + 4 * (size_t)n_q, 0u);
        rc = tsr_hip_msum_build_f16(m.f16.data(), n_kv, n_kv, n_q, m.words.data());
        if (rc < 0) return d->hip(rc, "mask summary");
        d->st.masks_summarized++;
    }
    return TSR_GG_OK;
}

int tsr_gg_buffer_get_tensor(tsr_gg_buffer * b, const tsr_gg_tensor * t, void * data, size_t offset, size_t size) {
    if (b == nullptr || t == nullptr || (size && data == nullptr)) return TSR_GG_E_ARG;
    tsr_gg_dev * d = b->dev;
    std::lock_guard<std::recursive_mutex> lk(d->mtx);
    uint64_t a;
    int rc = buf_enter(b, t, offset, size, &a);
    if (rc || size == 0) return rc;
    if (b->mode == kKv) rc = kv_access(d, b, a, size, nullptr, (uint8_t *)data, 0);
    else rc = d->hip(tsr_hip_read(d->ctx, data, b->mem + (a - b->vbase), size), t->name);
    if (rc) return rc;
    int32_t fl = 0;
    rc = tsr_hip_get_flags(d->ctx, &fl, 1);
    if (rc) return d->hip(rc, "device flags");
    if (fl) return d->fail(TSR_GG_E_FLAG, "a kernel raised device flags 0x%x (1: an index out of range, 2: an expired "
                                          "FLASH_ATTN_EXT wait, 4: an XCD placement check): the results are not valid", fl);
    return TSR_GG_OK;
}

int tsr_gg_buffer_memset_tensor(tsr_gg_buffer * b, const tsr_gg_tensor * t, uint8_t value, size_t offset, size_t size) {
    if (b == nullptr || t == nullptr) return TSR_GG_E_ARG;
    tsr_gg_dev * d = b->dev;
    std::lock_guard<std::recursive_mutex> lk(d->mtx);
    uint64_t a;
    int rc = buf_enter(b, t, offset, size, &a);
    if (rc || size == 0) return rc;
    if (b->mode == kKv) return kv_access(d, b, a, size, nullptr, nullptr, value);
    drop_weights_in(d, a, a + size);
    auto it = d->shadows.find(t->data);
    if (it != d->shadows.end() && offset < it->second.size())
        memset(it->second.data() + offset, value, std::min(size, it->second.size() - offset));
    return d->hip(tsr_hip_memset(d->ctx, b->mem + (a - b->vbase), value, size), t->name);
}

int tsr_gg_buffer_clear(tsr_gg_buffer * b, uint8_t value) {
    if (b == nullptr) return TSR_GG_E_ARG;
    tsr_gg_dev * d = b->dev;
    std::lock_guard<std::recursive_mutex> lk(d->mtx);
    uint64_t a;
    int rc = buf_enter(b, nullptr, 0, 0, &a);
    if (rc) return rc;
    if (b->mode == kKv) {
        for (const KvTensor & k : b->kv)
            if ((rc = kv_access(d, b, k.vaddr, k.nbytes, nullptr, nullptr, value)) != 0) return rc;
        return TSR_GG_OK;
    }
    drop_weights_in(d, b->vbase, b->vbase + b->size);
    return b->size ? d->hip(tsr_hip_memset(d->ctx, b->mem, value, b->size), "buffer clear") : TSR_GG_OK;
}

int tsr_gg_buffer_cpy_tensor(tsr_gg_buffer * b, const tsr_gg_tensor * src, const tsr_gg_tensor * dst) {
    if (b == nullptr || src == nullptr || dst == nullptr) return TSR_GG_E_ARG;
    tsr_gg_dev * d = b->dev;
    std::lock_guard<std::recursive_mutex> lk(d->mtx);
    if (d->ctx == nullptr) return 0;
    const size_t n = nbytes_of(d, src);
    if (n == 0 || n != nbytes_of(d, dst)) return 0;
    void *sp = nullptr, *dp = nullptr;
    std::string why;
    if (!dev_ptr(d, src->data, n, &sp, &why) || !dev_ptr(d, dst->data, n, &dp, &why)) return 0;
    drop_weights_in(d, dst->data, dst->data + n);
    d->shadows.erase(dst->data);                          // the host no longer knows the values
    d->masks.erase(dst->data);
    const int rc = tsr_hip_copy_async(d->ctx, dp, sp, n, d->stream);
    return rc ? d->hip(rc, "cpy_tensor") : 1;
}

int tsr_gg_buffer_free(tsr_gg_buffer * b) {
    if (b == nullptr) return TSR_GG_E_ARG;
    tsr_gg_dev * d = b->dev;
    std::lock_guard<std::recursive_mutex> lk(d->mtx);
    drop_plans(d);
    const uint64_t lo = b->vbase, hi = b->vbase + kVSpan;
    drop_weights_in(d, lo, hi);
    for (auto it = d->masks.begin(); it != d->masks.end();) it = it->first >= lo && it->first < hi ? d->masks.erase(it) : ++it;
    for (auto it = d->shadows.begin(); it != d->shadows.end();)
        it = it->first >= lo && it->first < hi ? d->shadows.erase(it) : ++it;
    if (d->ctx) {
        if (d->stream) tsr_hip_sync(d->ctx, d->stream);
        for (KvTensor & k : b->kv) if (k.kv) tsr_hip_kv_free(d->ctx, k.kv);
        if (b->mem) tsr_hip_free(d->ctx, b->mem);
    }
    d->buffers.erase(std::remove(d->buffers.begin(), d->buffers.end(), b), d->buffers.end());
    delete b;
    return TSR_GG_OK;
}

int tsr_gg_buffer_reset(tsr_gg_buffer * b) {
    if (b == nullptr) return TSR_GG_E_ARG;
    tsr_gg_dev * d = b->dev;
    std::lock_guard<std::recursive_mutex> lk(d->mtx);
    if (b->mode == kUndecided) b->tensors.clear();
    if (b->mode != kKv) {
        const uint64_t lo = b->vbase, hi = b->vbase + b->size;
        auto forget = [&](auto & m) {
            for (auto it = m.lower_bound(lo); it != m.end() && it->first < hi;) it = m.erase(it);
        };
        forget(d->masks);
        forget(d->shadows);
    }
    return TSR_GG_OK;
}

int tsr_gg_get_memory(tsr_gg_dev * d, size_t * free_bytes, size_t * total_bytes) {
    if (d == nullptr || free_bytes == nullptr || total_bytes == nullptr) return TSR_GG_E_ARG;
    std::lock_guard<std::recursive_mutex> lk(d->mtx);
    *free_bytes = *total_bytes = 0;
    if (d->ctx == nullptr) return TSR_GG_OK;
    size_t f = 0, t = 0;
    const int rc = tsr_hip_device_info(d->ctx, nullptr, nullptr, 0, &f, &t);
    if (rc) return d->hip(rc, "device memory");
    *free_bytes = f;
    *total_bytes = t;
    return TSR_GG_OK;
}

int tsr_gg_supports_op(tsr_gg_dev * d, const tsr_gg_tensor * op, char * why, size_t why_len) {
    if (d == nullptr || op == nullptr) return TSR_GG_E_ARG;
    std::lock_guard<std::recursive_mutex> lk(d->mtx);
    if (is_noop(op->op)) return 1;
    // the node alone, lowered as a one-node graph in describe mode; the fusion partners are judged by
    // the rules of their own position (MUL behind RMS_NORM, SCALE / TANH behind MUL_MAT)
    std::string w;
    bool ok = true;
    const tsr_gg_tensor * s0 = op->src[0];
    if (op->op == TSR_GG_OP_MUL) {
        const tsr_gg_tensor * o = s0 && s0->op == TSR_GG_OP_RMS_NORM ? op->src[1] : (op->src[1] && op->src[1]->op == TSR_GG_OP_RMS_NORM ? s0 : nullptr);
        if (o == nullptr) {
            ok = false;
            w = "MUL norm-weight: the weight multiply of an RMS_NORM's output, the only MUL the device runs [" +
                dims(op->src[0]) + " * " + dims(op->src[1]) + "]";
        } else if (o->type != TSR_GG_TYPE_F32 || o->ne[0] != op->ne[0] || !same_shape(op, op->src[0] == o ? op->src[1] : s0)) {
            ok = false;
            w = "MUL norm-weight: an f32 weight row as wide as the normalized rows [" + dims(o) + "]";
        }
    } else if (op->op == TSR_GG_OP_SCALE || op->op == TSR_GG_OP_UNARY) {
        const bool tanh_ok = op->op == TSR_GG_OP_SCALE || op->op_params[0] == TSR_GG_UNARY_TANH;
        const tsr_gg_tensor * up = s0;
        while (up && (up->op == TSR_GG_OP_SCALE || up->op == TSR_GG_OP_UNARY)) up = up->src[0];
        if (!tanh_ok || up == nullptr || up->op != TSR_GG_OP_MUL_MAT || (op->op == TSR_GG_OP_SCALE && param_f32(op, 1) != 0.0f)) {
            ok = false;
            w = "SCALE/TANH epilogue: only as the tail of a MUL_MAT, a SCALE or a softcap SCALE-TANH-SCALE chain [" +
                dims(op) + "]";
        }
    } else {
        Plan p;
        Lowerer L(d, false, &p);
        const tsr_gg_tensor * one[1] = {op};
        Graph g = make_graph(d, one, 1);
        int bad = -1;
        ok = L.lower(g, &bad);
        w = L.why;
    }
    if (!ok && why && why_len) snprintf(why, why_len, "%s", w.c_str());
    return ok ? 1 : 0;
}

int tsr_gg_lower(tsr_gg_dev * d, const tsr_gg_tensor * const * nodes, int n, tsr_gg_call * out, int cap, int * n_out) {
    if (d == nullptr || (n && nodes == nullptr) || n < 0 || n_out == nullptr || cap < 0) return TSR_GG_E_ARG;
    std::lock_guard<std::recursive_mutex> lk(d->mtx);
    Plan p;
    Lowerer L(d, false, &p);
    Graph g = make_graph(d, nodes, n);
    int bad = -1;
    const tsr_gg_stats saved = d->st;
    const bool ok = L.lower(g, &bad);
    d->st = saved;
    if (!ok) return d->fail(TSR_GG_E_UNSUPPORTED, "node %d '%s': %s", bad, bad >= 0 ? nodes[bad]->name : "?", L.why.c_str());
    *n_out = (int)p.calls.size();
    for (int i = 0; i < (int)p.calls.size() && i < cap; ++i) out[i] = p.calls[i].info;
    return TSR_GG_OK;
}

int tsr_gg_graph_compute(tsr_gg_dev * d, const tsr_gg_tensor * const * nodes, int n) {
    if (d == nullptr || (n && nodes == nullptr) || n < 0) return TSR_GG_E_ARG;
    std::lock_guard<std::recursive_mutex> lk(d->mtx);
    if (d->ctx == nullptr) return d->fail(TSR_GG_E_NODEV, "a probe device runs no graph");
    d->st.graphs++;
    const uint64_t key = tsr_gg_graph_key(nodes, n, d->epoch * 4 + d->options);
    auto it = d->plans.find(key);
    if (it == d->plans.end()) {
        d->st.plan_misses++;
        if (d->plans.size() >= kMaxPlans) {
            auto lru = d->plans.begin();
            for (auto j = d->plans.begin(); j != d->plans.end(); ++j) if (j->second.used < lru->second.used) lru = j;
            free_plan(d, lru->second);
            d->plans.erase(lru);
        }
        Plan p;
        Lowerer L(d, true, &p);
        Graph g = make_graph(d, nodes, n);
        int bad = -1;
        if (!L.lower(g, &bad)) {
            free_plan(d, p);
            return d->fail(TSR_GG_E_UNSUPPORTED, "node %d '%s': %s", bad, bad >= 0 ? nodes[bad]->name : "?", L.why.c_str());
        }
        bool changed = false;
        int rc = refresh_fa(d, p, &changed);
        if (rc == 0) rc = run_calls(d, p, nodes);
        d->st.calls += p.calls.size();
        d->st.eager_runs++;
        for (const Call & c : p.calls) d->st.fused += c.info.node2 >= 0;
        if (rc) {
            free_plan(d, p);
            return rc;
        }
        p.used = ++d->stamp;
        p.runs = 1;
        d->plans.emplace(key, std::move(p));
        return TSR_GG_OK;
    }
    Plan & p = it->second;
    d->st.plan_hits++;
    p.used = ++d->stamp;
    bool changed = false;
    int rc = refresh_fa(d, p, &changed);
    if (rc) return rc;
    d->st.calls += p.calls.size();
    if (!p.capturable) {
        d->st.eager_runs++;
        return run_calls(d, p, nodes);
    }
    if (p.graph == nullptr || changed) {
        if ((rc = capture(d, p)) != 0) return rc;
    }
    rc = tsr_hip_graph_launch(d->ctx, p.graph, d->stream);
    if (rc == TSR_HIP_E_ARG) {                          // the scratch moved since the capture
        if ((rc = capture(d, p)) != 0) return rc;
        rc = tsr_hip_graph_launch(d->ctx, p.graph, d->stream);
    }
    if (rc) return d->hip(rc, "graph launch");
    d->st.replays++;
    ++p.runs;
    return TSR_GG_OK;
}

int tsr_gg_synchronize(tsr_gg_dev * d) {
    if (d == nullptr) return TSR_GG_E_ARG;
    std::lock_guard<std::recursive_mutex> lk(d->mtx);
    if (d->ctx == nullptr) return TSR_GG_OK;
    int rc = tsr_hip_sync(d->ctx, d->stream);
    if (rc) return d->hip(rc, "synchronize");
    int32_t fl = 0;
    if ((rc = tsr_hip_get_flags(d->ctx, &fl, 1)) != 0) return d->hip(rc, "device flags");
    if (fl) return d->fail(TSR_GG_E_FLAG, "a kernel raised device flags 0x%x (1: an index out of range, 2: an expired "
                                          "FLASH_ATTN_EXT wait, 4: an XCD placement check): the results are not valid", fl);
    return TSR_GG_OK;
}

int tsr_gg_set_options(tsr_gg_dev * d, uint32_t options) {
    if (d == nullptr || (options & ~TSR_GG_OPT_NO_FUSION)) return TSR_GG_E_ARG;
    std::lock_guard<std::recursive_mutex> lk(d->mtx);
    d->options = options;
    return TSR_GG_OK;
}

int tsr_gg_get_stats(tsr_gg_dev * d, tsr_gg_stats * out) {
    if (d == nullptr || out == nullptr) return TSR_GG_E_ARG;
    std::lock_guard<std::recursive_mutex> lk(d->mtx);
    *out = d->st;
    return TSR_GG_OK;
}

int tsr_gg_kv_parse_name(const char * name, uint32_t * which, int * layer) { return kv_parse_name(name, which, layer) ? 1 : 0; }

uint64_t tsr_gg_graph_key(const tsr_gg_tensor * const * nodes, int n, uint64_t salt) {
    uint64_t h = mix(0x243F6A8885A308D3ull, salt);
    for (int i = 0; i < n; ++i) {
        const tsr_gg_tensor * t = nodes[i];
        h = key_tensor(h, t);
        for (int p = 0; p < 16; ++p) h = mix(h, (uint64_t)(uint32_t)t->op_params[p]);
        for (int s = 0; s < 10; ++s) {
            if (t->src[s] == nullptr) { h = mix(h, 0x5A5Aull + (uint64_t)s); continue; }
            h = key_tensor(h, t->src[s]);
        }
        h = mix(h, t->view_src ? t->view_src->data : 0);
    }
    return h;
}

int tsr_gg_quantize_q8_0(const float * x, int64_t K, void * blocks) {
    if (x == nullptr || blocks == nullptr || K < 0 || K % 32 != 0) return TSR_GG_E_ARG;
    quantize_q8_0(x, K, (uint8_t *)blocks);
    return TSR_GG_OK;
}

}  // extern "C"
