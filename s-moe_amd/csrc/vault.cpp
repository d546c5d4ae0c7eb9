// vault.cpp -- .smoe vault reader and HBM-resident expert pool loader.
//
// The reference streams expert blobs from the vault into a ring of host
// slots on demand (src/io/streamer.cpp) and learns the blob layout from
// expert 0's descriptors alone (main.cpp:167-198).  Here every blob of every
// MoE layer is copied once into one device pool, pool + (m * E + e) * stride
// for the m-th MoE layer, which is the layout the decode and prefill entry
// points take; every expert's table entry and tensor descriptors are checked
// against that common layout first.
//
// On-disk format (common.hpp:57-181, written by shatter_moe.py:947-1098):
//   [0]            SmoeHeader, 64 bytes (magic, version 1..2, table/data offsets,
//                  group size, bits, d_model, ...; reserved_ext = arch offset in v2)
//   table_offset   total_experts x ExpertEntry (48 bytes): layer id, expert id,
//                  absolute blob offset, raw and page-padded sizes
//   then           total_experts x 3 TensorDescriptor (44 bytes): gate, up, down
//   reserved_ext   (v2) SmoeArchBlock, 128 bytes, "SARC"
//   data_offset    blobs, each 16 KB aligned: [gate p][gate s][up p][up s][down p][down s]
// The header and arch-block checks follow main.cpp:96-157 and
// streamer.cpp:183-206.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <thread>
#include <vector>

#include <hip/hip_runtime.h>

#include "smoe_hip.h"

namespace {

#pragma pack(push, 1)
struct VHeader {
    uint8_t magic[8];
    uint32_t version, num_moe_layers, max_experts_per_layer, total_experts;
    uint64_t table_offset, data_offset;
    uint32_t group_size, bits, d_model, vocab_size, ffn_dim, reserved_ext;
};
struct VArch {
    uint8_t magic[4];
    uint32_t block_version, block_size, flags;
    float rope_theta;
    uint32_t num_heads, num_kv_heads, head_dim, moe_top_k, moe_ffn_dim, dense_ffn_dim, shared_expert_ffn_dim;
    uint32_t activation, num_hidden_layers;
    float rms_norm_eps;
    char model_type[24];
    uint8_t reserved[44];
};
struct VEntry {
    uint32_t layer_id, expert_id;
    uint64_t byte_offset, raw_size, padded_size;
    uint32_t group_size;
    uint64_t num_groups;
    uint8_t reserved[4];
};
struct VDesc {
    uint8_t tensor_type, ndim, reserved_0[2];
    uint32_t rows, cols;
    uint64_t packed_offset, packed_size, scales_offset, scales_size;
};
#pragma pack(pop)
static_assert(sizeof(VHeader) == 64, "SmoeHeader is 64 bytes");
static_assert(sizeof(VArch) == 128, "SmoeArchBlock is 128 bytes");
static_assert(sizeof(VEntry) == 48, "ExpertEntry is 48 bytes");
static_assert(sizeof(VDesc) == 44, "TensorDescriptor is 44 bytes");

constexpr uint8_t kMagic[8] = {'S', 'M', 'O', 'E', 0xDE, 0xEA, 0x00, 0x01};
constexpr uint8_t kArchMagic[4] = {'S', 'A', 'R', 'C'};
constexpr uint32_t kVersionMin = 1, kVersionMax = 2;
constexpr uint64_t kPage = 16384;          // blob alignment of the writer
constexpr uint32_t kMaxActive = 16;        // scout.hpp:32
constexpr size_t kStageBytes = 64u << 20;  // pinned staging buffer (two of them)
constexpr size_t kReadSlice = 8u << 20;    // one reader thread per slice of a staging fill
constexpr unsigned kReaders = 8;

thread_local std::string g_vault_err;

int fail(int code, const char* fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_vault_err = buf;
    return code;
}

bool read_at(int fd, void* dst, size_t n, uint64_t off)
{
    auto* p = static_cast<uint8_t*>(dst);
    while (n) {
        const ssize_t r = ::pread(fd, p, n, static_cast<off_t>(off));
        if (r <= 0) return false;
        p += r;
        n -= static_cast<size_t>(r);
        off += static_cast<uint64_t>(r);
    }
    return true;
}

// n bytes at off into dst, in up to kReaders slices read concurrently (a
// single pread from the page cache runs at ~16 GB/s, below PCIe)
bool read_parallel(int fd, void* dst, size_t n, uint64_t off)
{
    const unsigned k = static_cast<unsigned>(std::min<size_t>(kReaders, (n + kReadSlice - 1) / kReadSlice));
    if (k <= 1) return read_at(fd, dst, n, off);
    const size_t part = (n + k - 1) / k;
    bool ok[kReaders];
    std::vector<std::thread> th;
    for (unsigned i = 0; i < k; ++i) {
        const size_t b = i * part, len = std::min(part, n - std::min(n, b));
        ok[i] = true;
        if (len) th.emplace_back([&, i, b, len] { ok[i] = read_at(fd, static_cast<uint8_t*>(dst) + b, len, off + b); });
    }
    for (auto& t : th) t.join();
    for (unsigned i = 0; i < k; ++i)
        if (!ok[i]) return false;
    return true;
}

}  // namespace

struct SmoeVault {
    std::string path;
    uint64_t file_size = 0;
    VHeader hdr{};
    VArch arch{};
    bool arch_valid = false;
    std::vector<VEntry> table;
    std::vector<VDesc> descs;
    std::vector<uint32_t> layer_ids;   // distinct MoE layer ids, ascending
    std::vector<uint32_t> slot;        // table index of (m, e) at m * E + e
    SmoeVaultInfo info{};
};

extern "C" const char* smoe_hip_vault_error(void)
{
    return g_vault_err.c_str();
}

extern "C" int smoe_hip_vault_open(const char* path, SmoeVault** out)
{
    if (!path || !out) return fail(SMOE_ERR_ARG, "vault: NULL argument");
    *out = nullptr;
    const int fd = ::open(path, O_RDONLY);
    if (fd < 0) return fail(SMOE_ERR_VAULT, "vault: cannot open %s", path);
    struct Closer {
        int fd;
        ~Closer() { ::close(fd); }
    } closer{fd};
    struct stat st {};
    if (::fstat(fd, &st) != 0) return fail(SMOE_ERR_VAULT, "vault: cannot stat %s", path);
    auto v = std::make_unique<SmoeVault>();
    v->path = path;
    v->file_size = static_cast<uint64_t>(st.st_size);
    VHeader& h = v->hdr;

    // header (main.cpp:105-123, streamer.cpp:185-198)
    if (v->file_size < sizeof(VHeader) || !read_at(fd, &h, sizeof(h), 0))
        return fail(SMOE_ERR_VAULT, "vault: too small to be a .smoe file");
    if (std::memcmp(h.magic, kMagic, sizeof(kMagic)) != 0)
        return fail(SMOE_ERR_VAULT, "vault: invalid magic bytes, not a .smoe vault");
    if (h.version < kVersionMin || h.version > kVersionMax)
        return fail(SMOE_ERR_VAULT, "vault: version %u, supported %u-%u", h.version, kVersionMin, kVersionMax);
    if (h.total_experts == 0) return fail(SMOE_ERR_VAULT, "vault: contains zero experts");
    if (h.bits != 4) return fail(SMOE_ERR_BITS, "vault: %u-bit experts (only SMOE-Q4 is implemented)", h.bits);
    if (h.group_size != 64) return fail(SMOE_ERR_SHAPE, "vault: group size %u (SMOE-Q4 uses 64)", h.group_size);
    const uint64_t table_bytes = uint64_t(h.total_experts) * sizeof(VEntry);
    const uint64_t desc_bytes = uint64_t(h.total_experts) * 3 * sizeof(VDesc);
    // (every bound below is checked in subtraction form: sums of file-supplied
    // 64-bit values could wrap)
    if (h.table_offset < sizeof(VHeader) || h.data_offset > v->file_size || h.table_offset > h.data_offset ||
        table_bytes + desc_bytes > h.data_offset - h.table_offset)
        return fail(SMOE_ERR_VAULT, "vault: expert table [%llu, +%llu) does not fit before data offset %llu",
                    (unsigned long long)h.table_offset, (unsigned long long)(table_bytes + desc_bytes),
                    (unsigned long long)h.data_offset);

    // v2 arch block (main.cpp:125-157): required, checked, never guessed
    if (h.version >= 2) {
        if (h.reserved_ext == 0 || h.data_offset < sizeof(VArch) || h.reserved_ext > h.data_offset - sizeof(VArch))
            return fail(SMOE_ERR_VAULT, "vault: v2 vault has no valid arch-block offset");
        if (!read_at(fd, &v->arch, sizeof(VArch), h.reserved_ext) ||
            std::memcmp(v->arch.magic, kArchMagic, 4) != 0 || v->arch.block_size != sizeof(VArch) ||
            v->arch.block_version != 1)
            return fail(SMOE_ERR_VAULT, "vault: corrupt arch block in v2 vault");
        const VArch& a = v->arch;
        if (a.activation != 0)
            return fail(SMOE_ERR_VAULT, "vault: activation id %u (SiLU only)", a.activation);
        if (a.moe_top_k == 0 || a.moe_top_k > kMaxActive || a.head_dim == 0 || a.head_dim > 256 ||
            a.num_heads == 0 || a.num_kv_heads == 0 || a.num_heads % a.num_kv_heads != 0)
            return fail(SMOE_ERR_VAULT, "vault: arch block values out of engine limits (top_k=%u heads=%u/%u "
                        "head_dim=%u)", a.moe_top_k, a.num_heads, a.num_kv_heads, a.head_dim);
        v->arch_valid = true;
    }

    // table and descriptors (streamer.cpp:200-212 reads the table; the
    // descriptors follow it, main.cpp:170-175)
    v->table.resize(h.total_experts);
    v->descs.resize(size_t(h.total_experts) * 3);
    if (!read_at(fd, v->table.data(), table_bytes, h.table_offset) ||
        !read_at(fd, v->descs.data(), desc_bytes, h.table_offset + table_bytes))
        return fail(SMOE_ERR_VAULT, "vault: failed to read the expert table");

    // every expert against expert 0's layout
    const VDesc* d0 = &v->descs[0];
    const uint32_t I = d0[0].rows, D = d0[0].cols;
    if (I == 0 || D == 0) return fail(SMOE_ERR_SHAPE, "vault: empty expert matrices");
    const VEntry& e0 = v->table[0];
    std::map<uint32_t, std::vector<int64_t>> by_layer;
    for (uint32_t i = 0; i < h.total_experts; ++i) {
        const VEntry& e = v->table[i];
        const VDesc* dd = &v->descs[size_t(i) * 3];
        if (e.byte_offset < h.data_offset || e.byte_offset % kPage != 0 || e.raw_size > e.padded_size ||
            e.padded_size % kPage != 0 || e.byte_offset > v->file_size || e.raw_size > v->file_size - e.byte_offset)
            return fail(SMOE_ERR_VAULT, "vault: blob of layer %u expert %u at %llu (+%llu) is misplaced", e.layer_id,
                        e.expert_id, (unsigned long long)e.byte_offset, (unsigned long long)e.raw_size);
        if (e.raw_size != e0.raw_size || e.padded_size != e0.padded_size)
            return fail(SMOE_ERR_VAULT, "vault: layer %u expert %u has a different blob size", e.layer_id,
                        e.expert_id);
        for (int t = 0; t < 3; ++t) {
            const VDesc& x = dd[t];
            const uint32_t want_rows = t == 2 ? D : I, want_cols = t == 2 ? I : D;
            const uint64_t n = uint64_t(x.rows) * x.cols;
            if (x.tensor_type != t || x.ndim != 2 || x.rows != want_rows || x.cols != want_cols ||
                x.packed_size != n / 2 || x.scales_size != n / h.group_size * 2 || n % h.group_size != 0 ||
                x.packed_offset > e.raw_size || x.packed_size > e.raw_size - x.packed_offset ||
                x.scales_offset > e.raw_size || x.scales_size > e.raw_size - x.scales_offset)
                return fail(SMOE_ERR_VAULT, "vault: descriptor %d of layer %u expert %u does not describe a %ux%u "
                            "SMOE-Q4 matrix inside its blob", t, e.layer_id, e.expert_id, want_rows, want_cols);
            // the kernels read packed rows with 16-byte loads and scales as fp16
            if (x.packed_offset % 16 != 0 || x.scales_offset % 2 != 0)
                return fail(SMOE_ERR_VAULT, "vault: descriptor %d of layer %u expert %u: tensor offsets not aligned "
                            "(packed %% 16, scales %% 2)", t, e.layer_id, e.expert_id);
            if (x.packed_offset != d0[t].packed_offset || x.scales_offset != d0[t].scales_offset)
                return fail(SMOE_ERR_VAULT, "vault: layer %u expert %u lays its tensors out unlike expert 0",
                            e.layer_id, e.expert_id);
        }
        auto& slots = by_layer[e.layer_id];
        if (e.expert_id >= h.max_experts_per_layer)
            return fail(SMOE_ERR_VAULT, "vault: expert id %u >= max_experts_per_layer %u", e.expert_id,
                        h.max_experts_per_layer);
        if (slots.empty()) slots.assign(h.max_experts_per_layer, -1);
        if (slots[e.expert_id] >= 0)
            return fail(SMOE_ERR_VAULT, "vault: layer %u expert %u appears twice", e.layer_id, e.expert_id);
        slots[e.expert_id] = i;
    }
    if (h.d_model != 0 && h.d_model != D)
        return fail(SMOE_ERR_SHAPE, "vault: header d_model %u but expert matrices have %u columns", h.d_model, D);
    const uint32_t E = h.max_experts_per_layer;
    for (auto& [lid, slots] : by_layer) {
        for (uint32_t e = 0; e < E; ++e)
            if (slots[e] < 0)
                return fail(SMOE_ERR_VAULT, "vault: layer %u lacks expert %u (the pool needs every expert)", lid, e);
        v->layer_ids.push_back(lid);
        for (uint32_t e = 0; e < E; ++e) v->slot.push_back(static_cast<uint32_t>(slots[e]));
    }
    if (h.num_moe_layers != v->layer_ids.size())
        return fail(SMOE_ERR_VAULT, "vault: header says %u MoE layers, table holds %zu", h.num_moe_layers,
                    v->layer_ids.size());

    SmoeVaultInfo& f = v->info;
    f.version = h.version;
    f.num_moe_layers = h.num_moe_layers;
    f.experts_per_layer = E;
    f.total_experts = h.total_experts;
    f.group_size = h.group_size;
    f.bits = h.bits;
    f.d_model = D;
    f.d_ff = I;
    f.vocab_size = h.vocab_size;
    f.ffn_dim = h.ffn_dim;
    f.blob_bytes = e0.raw_size;
    f.stride = e0.padded_size;
    f.gate_packed_offset = d0[0].packed_offset;
    f.gate_scales_offset = d0[0].scales_offset;
    f.up_packed_offset = d0[1].packed_offset;
    f.up_scales_offset = d0[1].scales_offset;
    f.down_packed_offset = d0[2].packed_offset;
    f.down_scales_offset = d0[2].scales_offset;
    f.arch_valid = v->arch_valid ? 1u : 0u;
    if (v->arch_valid) {
        const VArch& a = v->arch;
        f.arch_flags = a.flags;
        f.num_heads = a.num_heads;
        f.num_kv_heads = a.num_kv_heads;
        f.head_dim = a.head_dim;
        f.moe_top_k = a.moe_top_k;
        f.moe_ffn_dim = a.moe_ffn_dim;
        f.dense_ffn_dim = a.dense_ffn_dim;
        f.shared_expert_ffn_dim = a.shared_expert_ffn_dim;
        f.num_hidden_layers = a.num_hidden_layers;
        f.rope_theta = a.rope_theta;
        f.rms_norm_eps = a.rms_norm_eps;
        std::memcpy(f.model_type, a.model_type, sizeof(f.model_type));
        f.model_type[sizeof(f.model_type) - 1] = 0;
    }
    *out = v.release();
    g_vault_err.clear();
    return SMOE_OK;
}

extern "C" void smoe_hip_vault_close(SmoeVault* v)
{
    delete v;
}

extern "C" int smoe_hip_vault_info(const SmoeVault* v, SmoeVaultInfo* info)
{
    if (!v || !info) return fail(SMOE_ERR_ARG, "vault: NULL argument");
    *info = v->info;
    return SMOE_OK;
}

extern "C" int smoe_hip_vault_layer_id(const SmoeVault* v, uint32_t moe_index, uint32_t* layer_id)
{
    if (!v || !layer_id) return fail(SMOE_ERR_ARG, "vault: NULL argument");
    if (moe_index >= v->layer_ids.size())
        return fail(SMOE_ERR_ARG, "vault: MoE layer %u of %zu", moe_index, v->layer_ids.size());
    *layer_id = v->layer_ids[moe_index];
    return SMOE_OK;
}

extern "C" int smoe_hip_vault_layer(const SmoeVault* v, uint32_t moe_index, const void* dev_pool,
                                    SmoeMoeLayer* layer)
{
    if (!v || !dev_pool || !layer) return fail(SMOE_ERR_ARG, "vault: NULL argument");
    if (moe_index >= v->layer_ids.size())
        return fail(SMOE_ERR_ARG, "vault: MoE layer %u of %zu", moe_index, v->layer_ids.size());
    const SmoeVaultInfo& f = v->info;
    layer->experts = static_cast<const uint8_t*>(dev_pool) + uint64_t(moe_index) * f.experts_per_layer * f.stride;
    layer->expert_stride = f.stride;
    layer->gate_packed_offset = f.gate_packed_offset;
    layer->gate_scales_offset = f.gate_scales_offset;
    layer->up_packed_offset = f.up_packed_offset;
    layer->up_scales_offset = f.up_scales_offset;
    layer->down_packed_offset = f.down_packed_offset;
    layer->down_scales_offset = f.down_scales_offset;
    return SMOE_OK;
}

extern "C" int smoe_hip_vault_load(const SmoeVault* v, void* dev_pool, uint64_t pool_bytes, void* hip_stream)
{
    if (!v || !dev_pool) return fail(SMOE_ERR_ARG, "vault: NULL argument");
    const SmoeVaultInfo& f = v->info;
    const uint64_t need = uint64_t(f.num_moe_layers) * f.experts_per_layer * f.stride;
    if (pool_bytes < need)
        return fail(SMOE_ERR_CAPACITY, "vault: pool of %llu bytes, the vault needs %llu",
                    (unsigned long long)pool_bytes, (unsigned long long)need);
    // copy segments: runs of pool slots whose blobs also follow each other in
    // the file (the writer's layer-major order makes the whole data region
    // one segment)
    struct Seg {
        uint64_t file_off, pool_off, bytes;
    };
    std::vector<Seg> segs;
    for (size_t s = 0; s < v->slot.size(); ++s) {
        const VEntry& e = v->table[v->slot[s]];
        const uint64_t pool_off = uint64_t(s) * f.stride;
        // a whole padded slot when the file holds it, else the blob alone
        const uint64_t n = e.byte_offset + f.stride <= v->file_size ? f.stride : f.blob_bytes;
        if (!segs.empty() && segs.back().bytes % f.stride == 0 &&
            segs.back().file_off + segs.back().bytes == e.byte_offset &&
            segs.back().pool_off + segs.back().bytes == pool_off)
            segs.back().bytes += n;
        else
            segs.push_back({e.byte_offset, pool_off, n});
    }
    const int fd = ::open(v->path.c_str(), O_RDONLY);
    if (fd < 0) return fail(SMOE_ERR_VAULT, "vault: cannot open %s", v->path.c_str());
    hipStream_t stream = static_cast<hipStream_t>(hip_stream);
    void* stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    int rc = SMOE_OK;
    auto hip_fail = [&](hipError_t e, const char* what) {
        rc = fail(SMOE_ERR_HIP, "vault: %s: %s", what, hipGetErrorString(e));
        return false;
    };
    bool ok = true;
    for (int i = 0; ok && i < 2; ++i) {
        hipError_t e = hipHostMalloc(&stage[i], kStageBytes, hipHostMallocDefault);
        if (e != hipSuccess) ok = hip_fail(e, "hipHostMalloc");
        else if ((e = hipEventCreateWithFlags(&done[i], hipEventDisableTiming)) != hipSuccess)
            ok = hip_fail(e, "hipEventCreate");
    }
    // double-buffered: fill one pinned buffer from the file while the other
    // is copied to the device
    int buf = 0;
    bool pending[2] = {false, false};
    for (size_t k = 0; ok && k < segs.size(); ++k) {
        for (uint64_t done_bytes = 0; ok && done_bytes < segs[k].bytes;) {
            const uint64_t n = std::min<uint64_t>(kStageBytes, segs[k].bytes - done_bytes);
            if (pending[buf]) {
                const hipError_t e = hipEventSynchronize(done[buf]);
                if (e != hipSuccess) { ok = hip_fail(e, "hipEventSynchronize"); break; }
                pending[buf] = false;
            }
            if (!read_parallel(fd, stage[buf], n, segs[k].file_off + done_bytes)) {
                rc = fail(SMOE_ERR_VAULT, "vault: read of %llu bytes at %llu failed", (unsigned long long)n,
                          (unsigned long long)(segs[k].file_off + done_bytes));
                ok = false;
                break;
            }
            hipError_t e = hipMemcpyAsync(static_cast<uint8_t*>(dev_pool) + segs[k].pool_off + done_bytes,
                                          stage[buf], n, hipMemcpyHostToDevice, stream);
            if (e != hipSuccess) { ok = hip_fail(e, "hipMemcpyAsync"); break; }
            if ((e = hipEventRecord(done[buf], stream)) != hipSuccess) { ok = hip_fail(e, "hipEventRecord"); break; }
            pending[buf] = true;
            done_bytes += n;
            buf ^= 1;
        }
    }
    for (int i = 0; i < 2; ++i)
        if (pending[i]) {
            const hipError_t e = hipEventSynchronize(done[i]);
            if (e != hipSuccess && rc == SMOE_OK) hip_fail(e, "hipEventSynchronize");
        }
    for (int i = 0; i < 2; ++i) {
        if (done[i]) (void)hipEventDestroy(done[i]);
        if (stage[i]) (void)hipHostFree(stage[i]);
    }
    ::close(fd);
    if (rc == SMOE_OK) g_vault_err.clear();
    return rc;
}
