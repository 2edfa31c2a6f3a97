// .qwenbin v2 reader / writer (host code).
//
// Reference: the container of include/config.cuh:107-172, read by
// QwenEngine::load_model_file and setup_arena (src/engine.cu:85-348), written
// by tools/export_qwen25.py:218-419.  The reader checks what the reference
// checks (magic, version, quant type, layer types, table bounds) and, beyond
// it, that every tensor the engine will use lies inside the file with the
// alignment the fast kernels need, so a bad file fails on the host with a
// named field instead of faulting on the device.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdio>
#include <cmath>
#include <cstring>

#include "qe_common.hpp"
#include "qwenbin_internal.hpp"

namespace qe {

MappedFile::~MappedFile() {
    if (data_ != nullptr) munmap(const_cast<uint8_t*>(data_), size_);
    if (fd_ >= 0) ::close(fd_);
}

int MappedFile::open(const char* path) {
    fd_ = ::open(path, O_RDONLY);
    if (fd_ < 0) return fail(QE_ERR_INVALID_ARGUMENT, "qwenbin: cannot open '%s': %s", path, std::strerror(errno));
    struct stat st {};
    if (fstat(fd_, &st) != 0) return fail(QE_ERR_INVALID_ARGUMENT, "qwenbin: cannot stat '%s'", path);
    size_ = static_cast<size_t>(st.st_size);
    if (size_ == 0) return fail(QE_ERR_INVALID_ARGUMENT, "qwenbin: '%s' is empty", path);
    void* p = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
    if (p == MAP_FAILED) return fail(QE_ERR_INVALID_ARGUMENT, "qwenbin: mmap of '%s' failed", path);
    data_ = static_cast<const uint8_t*>(p);
    return QE_OK;
}

namespace {

struct Checker {
    const QwenbinModel& m;
    uint64_t size;
    // tensor [off, off + bytes) inside the payload; `align` relative to weights_offset
    int tensor(const char* what, int layer, uint64_t off, uint64_t bytes, uint64_t align, bool required) const {
        if (off == 0) {
            if (!required) return QE_OK;
            return fail(QE_ERR_INVALID_ARGUMENT, "qwenbin: %s%s%d missing (offset 0)", what,
                        layer >= 0 ? " of layer " : "", layer);
        }
        const uint64_t w0 = m.header.weights_offset;
        if (off < w0 || off > size || bytes > size - off)
            return fail(QE_ERR_INVALID_ARGUMENT, "qwenbin: %s (layer %d) at %llu + %llu bytes is outside the payload "
                        "[%llu, %llu)", what, layer, static_cast<unsigned long long>(off),
                        static_cast<unsigned long long>(bytes), static_cast<unsigned long long>(w0),
                        static_cast<unsigned long long>(size));
        if ((off - w0) % align != 0)
            return fail(QE_ERR_UNSUPPORTED, "qwenbin: %s (layer %d) at payload offset %llu is not %llu-byte aligned",
                        what, layer, static_cast<unsigned long long>(off - w0), static_cast<unsigned long long>(align));
        return QE_OK;
    }
    int mat(const char* what, int layer, uint64_t w_off, uint64_t s_off, uint64_t rows, uint64_t K) const {
        if (int rc = tensor(what, layer, w_off, rows * K / 2, 16, true)) return rc;
        return tensor(what, layer, s_off, rows * (K / 128) * 2, 2, true);
    }
};

}  // namespace

int qwenbin_parse(const MappedFile& file, QwenbinModel& m) {
    const uint64_t size = file.size();
    if (size < sizeof(qe_qwenbin_header))
        return fail(QE_ERR_INVALID_ARGUMENT, "qwenbin: %llu bytes is too small for a header",
                    static_cast<unsigned long long>(size));
    std::memcpy(&m.header, file.data(), sizeof(m.header));
    const qe_qwenbin_header& h = m.header;
    if (h.magic != QE_QWENBIN_MAGIC) return fail(QE_ERR_INVALID_ARGUMENT, "qwenbin: bad magic 0x%08x", h.magic);
    if (h.version != 2)
        return fail(QE_ERR_UNSUPPORTED, "qwenbin: format version %u (this build reads version 2)", h.version);
    if (h.quant_type != QE_QWENBIN_QUANT_W4A16_G128)
        return fail(QE_ERR_UNSUPPORTED, "qwenbin: quant_type %u (only W4A16_G128 = 1 is supported)", h.quant_type);
    const uint64_t L = h.num_layers, H = h.hidden_size, I = h.intermediate_size, NQ = h.num_attention_heads,
                   NKV = h.num_kv_heads, HD = h.head_dim, V = h.vocab_size;
    if (L == 0 || L > 4096 || H == 0 || H % 128 != 0 || I == 0 || I % 128 != 0 || HD != 128 || NQ == 0 || NKV == 0 ||
        NQ % NKV != 0 || NQ * HD != H || V == 0 || V > (1u << 24) || H > 16384 || I > 32768)
        return fail(QE_ERR_UNSUPPORTED,
                    "qwenbin: dimensions outside this build (hidden %llu, intermediate %llu, heads %llu/%llu x %llu, "
                    "vocab %llu, layers %llu)", static_cast<unsigned long long>(H),
                    static_cast<unsigned long long>(I), static_cast<unsigned long long>(NQ),
                    static_cast<unsigned long long>(NKV), static_cast<unsigned long long>(HD),
                    static_cast<unsigned long long>(V), static_cast<unsigned long long>(L));
    // the RMSNorm kernels use eps = 1e-6 (RMS_NORM_EPS, include/config.cuh:20), as the reference's do
    if (!(std::fabs(h.rms_norm_eps - 1e-6f) <= 1e-12f))
        return fail(QE_ERR_UNSUPPORTED, "qwenbin: rms_norm_eps %g is not supported (the kernels use 1e-6)",
                    static_cast<double>(h.rms_norm_eps));
    if (h.layer_table_offset < sizeof(qe_qwenbin_header) || h.layer_table_offset > size ||
        L * sizeof(qe_qwenbin_layer) > size - h.layer_table_offset)
        return fail(QE_ERR_INVALID_ARGUMENT, "qwenbin: truncated layer table (offset %llu, %llu layers, file %llu)",
                    static_cast<unsigned long long>(h.layer_table_offset), static_cast<unsigned long long>(L),
                    static_cast<unsigned long long>(size));
    if (h.weights_offset == 0 || h.weights_offset > size || h.weights_offset % 256 != 0)
        return fail(QE_ERR_INVALID_ARGUMENT, "qwenbin: weights_offset %llu (must be 256-aligned, inside the file)",
                    static_cast<unsigned long long>(h.weights_offset));
    m.layers.resize(L);
    std::memcpy(m.layers.data(), file.data() + h.layer_table_offset, L * sizeof(qe_qwenbin_layer));
    const Checker c{m, size};
    const uint64_t QD = NQ * HD, KVD = NKV * HD;
    if (int rc = c.mat("embed_tokens", -1, h.embed_tokens_offset, h.reserved[0], V, H)) return rc;
    if (int rc = c.tensor("final_norm", -1, h.final_norm_offset, H * 2, 2, true)) return rc;
    m.untied_lm_head = h.lm_head_offset != 0 && h.lm_head_offset != h.embed_tokens_offset;
    if (m.untied_lm_head)
        if (int rc = c.mat("lm_head", -1, h.lm_head_offset, h.reserved[1], V, H)) return rc;
    for (uint64_t l = 0; l < L; ++l) {
        const qe_qwenbin_layer& d = m.layers[l];
        const int li = static_cast<int>(l);
        if (d.type != QE_QWENBIN_LAYER_GQA)
            return fail(QE_ERR_UNSUPPORTED, "qwenbin: layer %d has type %u (only GQA = 0)", li, d.type);
        if (d.mlp_up_offset != 0 && d.mlp_up_offset != d.mlp_gate_offset)
            return fail(QE_ERR_UNSUPPORTED, "qwenbin: layer %d stores gate and up separately (interleaved expected)", li);
        if (int rc = c.tensor("input_layernorm", li, d.norm1_weight_offset, H * 2, 2, true)) return rc;
        if (int rc = c.tensor("post_attention_layernorm", li, d.norm2_weight_offset, H * 2, 2, true)) return rc;
        if (int rc = c.mat("q_proj", li, d.qkv_weight_offset, d.q_scale_offset, QD, H)) return rc;
        if (int rc = c.mat("k_proj", li, d.k_weight_offset, d.k_scale_offset, KVD, H)) return rc;
        if (int rc = c.mat("v_proj", li, d.v_weight_offset, d.v_scale_offset, KVD, H)) return rc;
        if (int rc = c.tensor("q_bias", li, d.q_bias_offset, QD * 2, 2, false)) return rc;
        if (int rc = c.tensor("k_bias", li, d.k_bias_offset, KVD * 2, 2, false)) return rc;
        if (int rc = c.tensor("v_bias", li, d.v_bias_offset, KVD * 2, 2, false)) return rc;
        if (int rc = c.mat("o_proj", li, d.attn_out_weight_offset, d.attn_out_scale_offset, H, QD)) return rc;
        if (int rc = c.mat("gate_up_proj", li, d.mlp_gate_offset, d.mlp_gate_scale_offset, 2 * I, H)) return rc;
        if (int rc = c.mat("down_proj", li, d.mlp_down_offset, d.mlp_down_scale_offset, H, I)) return rc;
    }
    qe_qwenbin_info& in = m.info;
    in.version = h.version;
    in.quant_type = h.quant_type;
    in.tie_word_embeddings = m.untied_lm_head ? 0u : 1u;
    in.hidden_size = static_cast<int32_t>(H);
    in.intermediate_size = static_cast<int32_t>(I);
    in.num_layers = static_cast<int32_t>(L);
    in.num_q_heads = static_cast<int32_t>(NQ);
    in.num_kv_heads = static_cast<int32_t>(NKV);
    in.head_dim = static_cast<int32_t>(HD);
    in.vocab_size = static_cast<int32_t>(V);
    in.max_seq_len = static_cast<int32_t>(h.max_seq_len);
    in.rms_norm_eps = h.rms_norm_eps;
    in.rope_theta = h.rope_theta;
    in.file_size = size;
    in.weights_offset = h.weights_offset;
    in.weights_bytes = size - h.weights_offset;
    return QE_OK;
}

QwenbinWriter::QwenbinWriter(int num_layers) : layers_(static_cast<size_t>(num_layers)) {
    const uint64_t table_end = 4096 + static_cast<uint64_t>(num_layers) * sizeof(qe_qwenbin_layer);
    weights_offset_ = (table_end + 255) & ~uint64_t{255};
    header_.magic = QE_QWENBIN_MAGIC;
    header_.version = 2;
    header_.num_layers = static_cast<uint32_t>(num_layers);
    header_.quant_type = QE_QWENBIN_QUANT_W4A16_G128;
    header_.layer_table_offset = 4096;
    header_.weights_offset = weights_offset_;
}

uint64_t QwenbinWriter::add(const void* bytes, size_t n) {
    const uint64_t off = weights_offset_ + payload_.size();
    const uint8_t* b = static_cast<const uint8_t*>(bytes);
    payload_.insert(payload_.end(), b, b + n);
    payload_.resize((payload_.size() + 255) & ~size_t{255}, 0);
    return off;
}

int QwenbinWriter::write(const char* path) const {
    std::FILE* f = std::fopen(path, "wb");
    if (f == nullptr) return fail(QE_ERR_INVALID_ARGUMENT, "qwenbin: cannot create '%s': %s", path, std::strerror(errno));
    std::vector<uint8_t> head(weights_offset_, 0);
    std::memcpy(head.data(), &header_, sizeof(header_));
    std::memcpy(head.data() + 4096, layers_.data(), layers_.size() * sizeof(qe_qwenbin_layer));
    const bool ok = std::fwrite(head.data(), 1, head.size(), f) == head.size() &&
                    std::fwrite(payload_.data(), 1, payload_.size(), f) == payload_.size();
    const bool closed = std::fclose(f) == 0;
    if (!ok || !closed) return fail(QE_ERR_INVALID_ARGUMENT, "qwenbin: write to '%s' failed", path);
    return QE_OK;
}

}  // namespace qe

extern "C" int qe_qwenbin_inspect(const char* path, qe_qwenbin_info* info) {
    QE_REQUIRE(path && info, "qwenbin_inspect: NULL argument");
    qe::MappedFile f;
    if (int rc = f.open(path)) return rc;
    qe::QwenbinModel m;
    if (int rc = qe::qwenbin_parse(f, m)) return rc;
    *info = m.info;
    qe::clear_error();
    return QE_OK;
}
