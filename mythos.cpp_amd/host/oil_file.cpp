// oil_file.cpp — `.oil` reader that repacks tensors into the kernels'
// structure-of-arrays layouts (include/mythos_oil_file.h).
//
// The reference's OILReader re-walks all preceding blocks on every
// read_block (src/oil_format.cpp:355-361, O(blocks^2) per tensor) and
// dequantises to FP32; here the file is indexed once at open and tensors stay
// quantised.  All reads are bounds-checked against the mapped size.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdarg>
#include <cstdio>
#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "mythos_oil_file.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

struct Block {
    uint32_t nw = 0;
    uint8_t format = 0;
    size_t cb_off = 0, cb_bytes = 0, idx_off = 0, idx_bytes = 0;
};

struct Tensor {
    std::string name;
    uint32_t start = 0, count = 0;
};

constexpr uint32_t kMagicOil8 = 0x4F494C38u, kMagicOil4 = 0x4F494C34u;

}  // namespace

struct mth_oil_file {
    const uint8_t* data = nullptr;
    size_t size = 0;
    std::vector<Block> blocks;
    std::vector<Tensor> tensors;

    bool get(size_t off, void* dst, size_t n) const {
        if (off > size || n > size - off) return false;
        std::memcpy(dst, data + off, n);
        return true;
    }
    const Tensor* find(const char* name) const {
        for (const Tensor& t : tensors)
            if (t.name == name) return &t;
        return nullptr;
    }
};

namespace {

int index_file(mth_oil_file* f) {
    char magic[4];
    uint32_t cfg = 0, nfmt = 0, nten = 0;
    if (!f->get(0, magic, 4) || std::memcmp(magic, "OIL1", 4) != 0) return fail(MTH_FILE_EFORMAT, "not an OIL1 file");
    if (!f->get(12, &cfg, 4)) return fail(MTH_FILE_EFORMAT, "truncated header");
    size_t p = 16 + (size_t)cfg;
    if (!f->get(p, &nfmt, 4)) return fail(MTH_FILE_EFORMAT, "truncated format table");
    p += 4;
    const size_t fmt_off = p;
    if ((size_t)nfmt * 9 > f->size - p) return fail(MTH_FILE_EFORMAT, "format table of %u entries past the end", nfmt);
    p += (size_t)nfmt * 9;
    if (!f->get(p, &nten, 4)) return fail(MTH_FILE_EFORMAT, "truncated tensor table");
    p += 4;
    f->tensors.resize(nten);
    for (uint32_t i = 0; i < nten; i++) {
        uint16_t len = 0;
        if (!f->get(p, &len, 2) || (size_t)len > f->size - p - 2)
            return fail(MTH_FILE_EFORMAT, "tensor entry %u truncated", i);
        f->tensors[i].name.assign((const char*)f->data + p + 2, len);
        p += 2 + len;
        if (!f->get(p, &f->tensors[i].start, 4) || !f->get(p + 4, &f->tensors[i].count, 4))
            return fail(MTH_FILE_EFORMAT, "tensor entry %u truncated", i);
        p += 8;
    }
    // blocks, in file order; block b's format comes from format entry b
    // (OILReader::read_block indexes the table by position)
    f->blocks.resize(nfmt);
    for (uint32_t b = 0; b < nfmt; b++) {
        Block& k = f->blocks[b];
        uint32_t cb = 0, ib = 0;
        f->get(fmt_off + (size_t)b * 9 + 4, &k.format, 1);
        if (!f->get(p, &k.nw, 4) || !f->get(p + 4, &cb, 4)) return fail(MTH_FILE_EFORMAT, "block %u truncated", b);
        k.cb_off = p + 8;
        k.cb_bytes = cb;
        if ((size_t)cb > f->size - k.cb_off || !f->get(k.cb_off + cb, &ib, 4))
            return fail(MTH_FILE_EFORMAT, "block %u truncated", b);
        k.idx_off = k.cb_off + cb + 4;
        k.idx_bytes = ib;
        if ((size_t)ib > f->size - k.idx_off) return fail(MTH_FILE_EFORMAT, "block %u indices past the end", b);
        p = k.idx_off + ib;
    }
    for (const Tensor& t : f->tensors)
        if ((uint64_t)t.start + t.count > nfmt)
            return fail(MTH_FILE_EFORMAT, "tensor '%s' refers to blocks past the table", t.name.c_str());
    return MTH_FILE_OK;
}

int fmt_of(uint8_t b) {
    return b <= 3 ? (int)b : MTH_OIL_FP32;
}

// Bytes one block of n weights needs in each layout.
size_t idx_need(int fmt, uint64_t n) {
    switch (fmt) {
        case MTH_OIL_OIL8: return n;
        case MTH_OIL_OIL4: return (n + 1) / 2;
        case MTH_OIL_TERNARY: return (n + 3) / 4;
        case MTH_OIL_BINARY: return (n + 7) / 8;
        default: return n * 4;
    }
}

// Per-element codes of a tensor in file order: OIL8 index bytes, OIL4 nibbles
// (each block's own even/odd nibble order, as OILReader::read_tensor walks
// them, src/oil_format.cpp:444-449), ternary 2-bit codes (element j of a
// block in bits 2(j%4) of its byte j/4, tools/convert.cpp:338-341).
int gather_codes(const mth_oil_file* f, const Tensor* t, int fm, uint8_t* out) {
    for (uint32_t b = t->start; b < t->start + t->count; b++) {
        const Block& k = f->blocks[b];
        if (k.idx_bytes < idx_need(fm, k.nw))
            return fail(MTH_FILE_EFORMAT, "block %u of '%s': short indices", b, t->name.c_str());
        const uint8_t* src = f->data + k.idx_off;
        for (uint32_t j = 0; j < k.nw; j++) {
            if (fm == MTH_OIL_OIL8) out[j] = src[j];
            else if (fm == MTH_OIL_OIL4) out[j] = (src[j >> 1] >> ((j & 1) * 4)) & 15;
            else out[j] = (src[j >> 2] >> ((j & 3) * 2)) & 3;
        }
        out += k.nw;
    }
    return MTH_FILE_OK;
}

// dst[r][c] = src[c][r] for a [cols][rows] source, in 64x64 tiles.
template <typename T>
void transpose(const T* src, T* dst, int64_t rows, int64_t cols) {
    for (int64_t c0 = 0; c0 < cols; c0 += 64)
        for (int64_t r0 = 0; r0 < rows; r0 += 64)
            for (int64_t r = r0; r < std::min(rows, r0 + 64); r++)
                for (int64_t c = c0; c < std::min(cols, c0 + 64); c++) dst[r * cols + c] = src[c * rows + r];
}

// Checks that every block of `t` carries the same codebook as its first.
bool same_codebooks(const mth_oil_file* f, const Tensor* t, size_t off, size_t n) {
    const Block& k0 = f->blocks[t->start];
    for (uint32_t b = t->start + 1; b < t->start + t->count; b++)
        if (std::memcmp(f->data + f->blocks[b].cb_off + off, f->data + k0.cb_off + off, n) != 0) return false;
    return true;
}

}  // namespace

extern "C" {

const char* mth_oil_error(void) { return g_err; }

mth_oil_file* mth_oil_open(const char* path) {
    if (!path) {
        fail(MTH_FILE_EINVAL, "mth_oil_open: null path");
        return nullptr;
    }
    const int fd = open(path, O_RDONLY);
    if (fd < 0) {
        fail(MTH_FILE_EINVAL, "mth_oil_open: cannot open %s", path);
        return nullptr;
    }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 16) {
        close(fd);
        fail(MTH_FILE_EFORMAT, "mth_oil_open: %s is too short", path);
        return nullptr;
    }
    void* m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) {
        fail(MTH_FILE_EINVAL, "mth_oil_open: cannot map %s", path);
        return nullptr;
    }
    mth_oil_file* f = new mth_oil_file;
    f->data = (const uint8_t*)m;
    f->size = (size_t)st.st_size;
    if (index_file(f) != MTH_FILE_OK) {
        mth_oil_close(f);
        return nullptr;
    }
    g_err[0] = '\0';
    return f;
}

void mth_oil_close(mth_oil_file* f) {
    if (!f) return;
    if (f->data) munmap((void*)f->data, f->size);
    delete f;
}

int64_t mth_oil_num_tensors(const mth_oil_file* f) { return f ? (int64_t)f->tensors.size() : 0; }

const char* mth_oil_tensor_name(const mth_oil_file* f, int64_t i) {
    if (!f || i < 0 || i >= (int64_t)f->tensors.size()) return nullptr;
    return f->tensors[(size_t)i].name.c_str();
}

int mth_oil_tensor_info(const mth_oil_file* f, const char* name, int* format, int64_t* num_weights,
                        int64_t* num_blocks, int64_t* block_weights) {
    if (!f || !name) return fail(MTH_FILE_EINVAL, "mth_oil_tensor_info: null argument");
    const Tensor* t = f->find(name);
    if (!t) return fail(MTH_FILE_EINVAL, "mth_oil_tensor_info: no tensor '%s'", name);
    int fm = -1;
    int64_t total = 0, bw = -2;
    for (uint32_t b = t->start; b < t->start + t->count; b++) {
        const Block& k = f->blocks[b];
        const int kf = fmt_of(k.format);
        if (fm >= 0 && kf != fm) return fail(MTH_FILE_EUNSUPPORTED, "tensor '%s' mixes block formats", name);
        fm = kf;
        total += k.nw;
        bw = (bw == -2 || bw == (int64_t)k.nw) ? (int64_t)k.nw : -1;
    }
    if (format) *format = fm;
    if (num_weights) *num_weights = total;
    if (num_blocks) *num_blocks = t->count;
    if (block_weights) *block_weights = bw < 0 ? -1 : bw;
    return MTH_FILE_OK;
}

int mth_oil_repack(const mth_oil_file* f, const char* name, int64_t rows, int64_t cols, int in_major,
                   void* indices, int64_t indices_bytes, void* codebooks, int64_t codebooks_bytes,
                   int64_t* cb_block) {
    int fm = 0;
    int64_t nw = 0, nb = 0, bw = 0;
    int rc = mth_oil_tensor_info(f, name, &fm, &nw, &nb, &bw);
    if (rc != MTH_FILE_OK) return rc;
    if (rows <= 0 || cols <= 0 || rows * cols != nw)
        return fail(MTH_FILE_EINVAL, "tensor '%s' has %lld weights, not %lld x %lld", name, (long long)nw,
                    (long long)rows, (long long)cols);
    if (!indices) return fail(MTH_FILE_EINVAL, "mth_oil_repack: null indices buffer");
    const Tensor* t = f->find(name);
    uint8_t* out = (uint8_t*)indices;
    const size_t need = idx_need(fm, (uint64_t)nw);
    if ((size_t)indices_bytes < need)
        return fail(MTH_FILE_EINVAL, "tensor '%s' needs %zu index bytes, buffer has %lld", name, need,
                    (long long)indices_bytes);
    if (cb_block) *cb_block = 0;
    if ((fm == MTH_OIL_OIL4 || fm == MTH_OIL_TERNARY) && cols % (fm == MTH_OIL_OIL4 ? 2 : 4) != 0)
        return fail(MTH_FILE_EUNSUPPORTED, "tensor '%s': rows of %lld weights do not end on a byte", name,
                    (long long)cols);

    // codebook checks, shared by both orientations
    if (fm == MTH_OIL_OIL4 || fm == MTH_OIL_OIL8) {
        const bool o4 = fm == MTH_OIL_OIL4;
        const uint32_t magic_want = o4 ? kMagicOil4 : kMagicOil8;
        const size_t cbn = o4 ? 32 : 1024;
        for (uint32_t b = t->start; b < t->start + t->count; b++) {
            uint32_t magic = 0;
            const Block& k = f->blocks[b];
            if (k.cb_bytes < 4 + cbn || !f->get(k.cb_off, &magic, 4) || magic != magic_want)
                return fail(MTH_FILE_EFORMAT, "block %u of '%s': not an %s codebook", b, name, o4 ? "OIL4" : "OIL8");
        }
        const bool one = same_codebooks(f, t, 4, cbn);
        if (!o4 && !one) return fail(MTH_FILE_EUNSUPPORTED, "tensor '%s': OIL8 blocks with different codebooks", name);
        if (o4 && in_major && !one)
            return fail(MTH_FILE_EUNSUPPORTED,
                        "tensor '%s': an input-major OIL4 tensor with per-block codebooks has no per-row layout", name);
        const int64_t ncb = (o4 && !in_major) ? nb : 1;
        if (!codebooks || codebooks_bytes < ncb * (int64_t)cbn)
            return fail(MTH_FILE_EINVAL, "tensor '%s' needs %lld codebook bytes", name, (long long)(ncb * cbn));
        if (o4 && !in_major && nb > 1 && (bw <= 0 || bw % 2 != 0 || cols % bw != 0))
            return fail(MTH_FILE_EUNSUPPORTED,
                        "tensor '%s': OIL4 blocks of %lld weights do not tile rows of %lld (need one length that "
                        "is even and divides the row)", name, (long long)bw, (long long)cols);
    }

    if (fm == MTH_OIL_FP32) {
        std::vector<float> tmp(in_major ? (size_t)nw : 0);
        float* dst = in_major ? tmp.data() : (float*)indices;
        for (uint32_t b = t->start; b < t->start + t->count; b++) {
            const Block& k = f->blocks[b];
            if (k.idx_bytes < (size_t)k.nw * 4) return fail(MTH_FILE_EFORMAT, "block %u of '%s': short data", b, name);
            f->get(k.idx_off, dst, (size_t)k.nw * 4);
            dst += k.nw;
        }
        if (in_major) transpose(tmp.data(), (float*)indices, rows, cols);
        return MTH_FILE_OK;
    }
    if (fm == MTH_OIL_BINARY)
        return fail(MTH_FILE_EUNSUPPORTED, "tensor '%s': binary blocks are not on the quantized path", name);

    if (fm == MTH_OIL_OIL4 && !in_major) {
        // blocks are whole nibble pairs: copy bytes, one codebook per block
        uint8_t* cbo = (uint8_t*)codebooks;
        for (uint32_t b = t->start; b < t->start + t->count; b++) {
            const Block& k = f->blocks[b];
            if (k.nw % 2 != 0 && nb > 1) return fail(MTH_FILE_EUNSUPPORTED, "tensor '%s': odd OIL4 block", name);
            if (k.idx_bytes < (size_t)k.nw / 2) return fail(MTH_FILE_EFORMAT, "block %u of '%s': short indices", b, name);
            f->get(k.cb_off + 4, cbo, 32);
            cbo += 32;
            f->get(k.idx_off, out, k.nw / 2);
            out += k.nw / 2;
        }
        if (cb_block) *cb_block = nb > 1 ? bw : 0;
        return MTH_FILE_OK;
    }
    if (fm == MTH_OIL_OIL8 && !in_major) {
        for (uint32_t b = t->start; b < t->start + t->count; b++) {
            const Block& k = f->blocks[b];
            if (k.idx_bytes < k.nw) return fail(MTH_FILE_EFORMAT, "block %u of '%s': short indices", b, name);
            f->get(k.idx_off, out, k.nw);
            out += k.nw;
        }
        f->get(f->blocks[t->start].cb_off + 4, codebooks, 1024);
        return MTH_FILE_OK;
    }

    // element-wise: ternary (either orientation), input-major OIL4 / OIL8
    std::vector<uint8_t> codes((size_t)nw), tr;
    rc = gather_codes(f, t, fm, codes.data());
    if (rc != MTH_FILE_OK) return rc;
    const uint8_t* c = codes.data();
    if (in_major) {
        tr.resize((size_t)nw);
        transpose(codes.data(), tr.data(), rows, cols);
        c = tr.data();
    }
    if (fm == MTH_OIL_OIL8) {
        std::memcpy(out, c, (size_t)nw);
    } else if (fm == MTH_OIL_OIL4) {
        for (int64_t i = 0; i < nw / 2; i++) out[i] = (uint8_t)(c[2 * i] | (c[2 * i + 1] << 4));
    } else {
        for (int64_t i = 0; i < nw / 4; i++)
            out[i] = (uint8_t)(c[4 * i] | (c[4 * i + 1] << 2) | (c[4 * i + 2] << 4) | (c[4 * i + 3] << 6));
    }
    if (fm == MTH_OIL_OIL4 || fm == MTH_OIL_OIL8)
        f->get(f->blocks[t->start].cb_off + 4, codebooks, fm == MTH_OIL_OIL4 ? 32 : 1024);
    else if (codebooks && codebooks_bytes >= 12 && f->blocks[t->start].cb_bytes >= 12)
        f->get(f->blocks[t->start].cb_off, codebooks, 12);
    return MTH_FILE_OK;
}

int mth_oil_upload(const mth_oil_file* f, const char* name, int64_t rows, int64_t cols, int in_major,
                   void* d_indices, int64_t indices_bytes, void* d_codebooks, int64_t codebooks_bytes,
                   int64_t* cb_block, void* stream) {
    int fm = 0;
    int64_t nw = 0, nb = 0, bw = 0;
    int rc = mth_oil_tensor_info(f, name, &fm, &nw, &nb, &bw);
    if (rc != MTH_FILE_OK) return rc;
    const size_t ib = idx_need(fm, (uint64_t)(rows * cols > 0 ? rows * cols : 0));
    const size_t cbb = fm == MTH_OIL_OIL4 ? (in_major ? 32 : (size_t)nb * 32)
                                          : (fm == MTH_OIL_OIL8 ? 1024 : (fm == MTH_OIL_TERNARY ? 12 : 0));
    std::vector<uint8_t> hi(ib), hc(cbb ? cbb : 1);
    rc = mth_oil_repack(f, name, rows, cols, in_major, hi.data(), (int64_t)ib, cbb ? hc.data() : nullptr,
                        (int64_t)cbb, cb_block);
    if (rc != MTH_FILE_OK) return rc;
    if ((size_t)indices_bytes < ib || (cbb && d_codebooks && (size_t)codebooks_bytes < cbb))
        return fail(MTH_FILE_EINVAL, "tensor '%s': device buffers too small (%zu + %zu bytes needed)", name, ib, cbb);
    hipStream_t s = (hipStream_t)stream;
    hipError_t e = hipMemcpyAsync(d_indices, hi.data(), ib, hipMemcpyHostToDevice, s);
    if (e == hipSuccess && cbb && d_codebooks) e = hipMemcpyAsync(d_codebooks, hc.data(), cbb, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return fail(MTH_FILE_EDEVICE, "tensor '%s': upload failed: %s", name, hipGetErrorString(e));
    return MTH_FILE_OK;
}

}  // extern "C"
