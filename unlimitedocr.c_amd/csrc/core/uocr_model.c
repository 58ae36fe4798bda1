/* uocr_model.c - .uocr reader/validator and decoder tensor binding. */
#define _FILE_OFFSET_BITS 64
#define _POSIX_C_SOURCE 200809L
#include "uocr_model.h"

#include <errno.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static int fail(char *err, size_t n, const char *fmt, ...) {
    if (err != NULL && n > 0u) {
        va_list ap;
        va_start(ap, fmt);
        (void)vsnprintf(err, n, fmt, ap);
        va_end(ap);
    }
    return -1;
}

static int in_range(uint64_t off, uint64_t len, uint64_t total) {
    return off <= total && len <= total - off;
}

static int in_section(uint64_t off, uint64_t len, const uocr_section_entry *s) {
    return s != NULL && off >= s->offset && in_range(off - s->offset, len, s->size);
}

static int nonzero32(const uint8_t h[32]) {
    for (int i = 0; i < 32; ++i) {
        if (h[i] != 0u) return 1;
    }
    return 0;
}

const char *uocr_qprofile_name(uint32_t q) {
    switch (q) {
        case UOCR_QPROFILE_FP16: return "fp16";
        case UOCR_QPROFILE_MIXED_Q8_0: return "mixed-q8_0";
        case UOCR_QPROFILE_MIXED_Q4: return "mixed-q4";
        default: return "unknown";
    }
}

const char *uocr_qtype_name(uint32_t q) {
    switch (q) {
        case UOCR_TENSOR_F16: return "f16";
        case UOCR_TENSOR_F32: return "f32";
        case UOCR_TENSOR_Q8_0: return "q8_0";
        case UOCR_TENSOR_Q4_0: return "q4_0";
        case UOCR_TENSOR_Q4_1: return "q4_1";
        default: return "unknown";
    }
}

static const uocr_section_entry *find_section(const uocr_file_header *h, const uocr_section_entry *s, uint32_t type) {
    for (uint32_t i = 0; i < h->section_count; ++i) {
        if (s[i].type == type) return &s[i];
    }
    return NULL;
}

/* config equality with the model constants (uocr_model_file.c:324-362) */
static int check_config(const uocr_config_record *c, char *err, size_t n) {
    const uint32_t expect[27] = {UOCR_VOCAB_SIZE, UOCR_BPE_VOCAB_SIZE, UOCR_ADDED_TOKEN_COUNT, (uint32_t)UOCR_TOKEN_BOS,
                                 (uint32_t)UOCR_TOKEN_EOS, (uint32_t)UOCR_TOKEN_PAD, (uint32_t)UOCR_TOKEN_IMAGE,
                                 UOCR_HIDDEN_SIZE, UOCR_DECODER_LAYERS, UOCR_ATTENTION_HEADS, UOCR_KV_HEADS,
                                 UOCR_HEAD_DIM, UOCR_ROPE_THETA, UOCR_MAX_POSITIONS, UOCR_GENERATED_RING_WINDOW,
                                 UOCR_DENSE_FIRST_LAYERS, UOCR_ROUTED_EXPERTS, UOCR_MOE_TOP_K,
                                 UOCR_MOE_EXPERT_INTERMEDIATE, UOCR_MOE_SHARED_EXPERTS,
                                 UOCR_DENSE_LAYER0_INTERMEDIATE, UOCR_PROJECTOR_IN_SIZE, UOCR_HIDDEN_SIZE,
                                 UOCR_VISION_PATCH_SIZE, UOCR_DOWNSAMPLE_RATIO, UOCR_GLOBAL_VIEW_SIZE,
                                 UOCR_LOCAL_VIEW_SIZE};
    static const char *names[27] = {"vocab_size", "bpe_vocab_size", "added_token_count", "bos_token_id",
                                    "eos_token_id", "pad_token_id", "image_token_id", "hidden_size",
                                    "decoder_layers", "attention_heads", "kv_heads", "head_dim", "rope_theta",
                                    "max_positions", "generated_ring_window", "dense_first_layers",
                                    "routed_experts", "moe_top_k", "moe_expert_intermediate", "shared_experts",
                                    "dense_layer0_intermediate", "projector_in", "projector_out",
                                    "vision_patch_size", "downsample_ratio", "supported_global_view",
                                    "supported_local_view"};
    uint32_t got[27];
    memcpy(got, c, sizeof(got));
    for (int i = 0; i < 27; ++i) {
        if (got[i] != expect[i]) return fail(err, n, "config.%s mismatch: got %u expected %u", names[i], got[i], expect[i]);
    }
    return 0;
}

static int check_tokenizer(const uint8_t *b, const uocr_section_entry *s, char *err, size_t n) {
    if (s == NULL) return 0;
    if (s->size < sizeof(uocr_tokenizer_metadata_record)) return fail(err, n, "tokenizer metadata section too small");
    const uocr_tokenizer_metadata_record *t = (const uocr_tokenizer_metadata_record *)(const void *)(b + s->offset);
    if (t->magic != UOCR_TOKENIZER_METADATA_MAGIC) return fail(err, n, "bad tokenizer metadata magic 0x%08x", t->magic);
    if (t->version != UOCR_FORMAT_VERSION) return fail(err, n, "unsupported tokenizer metadata version %u", t->version);
    if (t->record_size != sizeof(*t)) return fail(err, n, "unexpected tokenizer metadata record size %u", t->record_size);
    if ((t->flags & UOCR_TOKENIZER_FLAG_C_V1_NOT_REQUIRED) == 0u) {
        return fail(err, n, "tokenizer metadata must declare that C v1 does not require tokenizer tables");
    }
    if (!nonzero32(t->tokenizer_hash)) return fail(err, n, "tokenizer metadata hash is missing");
    if (t->vocab_size != UOCR_VOCAB_SIZE || t->eos_token_id != (uint32_t)UOCR_TOKEN_EOS ||
        t->image_token_id != (uint32_t)UOCR_TOKEN_IMAGE) {
        return fail(err, n, "tokenizer metadata disagrees with the model constants");
    }
    const int has = t->tokenizer_json_size != 0u;
    if (has != ((t->flags & UOCR_TOKENIZER_FLAG_EMBEDDED_PAYLOAD) != 0u)) {
        return fail(err, n, "tokenizer embedded-payload flag does not match payload size");
    }
    if (has && (!in_range(t->tokenizer_json_offset, t->tokenizer_json_size, s->size) ||
                t->tokenizer_json_offset < sizeof(*t))) {
        return fail(err, n, "tokenizer payload is outside its section");
    }
    if (!has && t->tokenizer_json_offset != 0u) return fail(err, n, "tokenizer payload offset set without payload size");
    return 0;
}

static int check_provenance(const uint8_t *b, const uocr_file_header *h, const uocr_section_entry *s,
                            uint32_t tensor_count, char *err, size_t n) {
    if (s == NULL) return 0;
    if (s->size < sizeof(uocr_provenance_record)) return fail(err, n, "provenance section too small");
    const uocr_provenance_record *p = (const uocr_provenance_record *)(const void *)(b + s->offset);
    if (p->magic != UOCR_PROVENANCE_MAGIC) return fail(err, n, "bad provenance magic 0x%08x", p->magic);
    if (p->version != UOCR_FORMAT_VERSION) return fail(err, n, "unsupported provenance version %u", p->version);
    if (p->record_size != sizeof(*p)) return fail(err, n, "unexpected provenance record size %u", p->record_size);
    if (p->qprofile != h->qprofile) return fail(err, n, "provenance qprofile mismatch: got %u expected %u", p->qprofile, h->qprofile);
    if (!nonzero32(p->config_hash) || !nonzero32(p->tokenizer_hash) || !nonzero32(p->safetensors_index_hash)) {
        return fail(err, n, "provenance hashes are missing");
    }
    const uint64_t acc = (uint64_t)p->runtime_tensor_count + p->preserved_unused_tensor_count + p->omitted_tensor_count;
    if (acc != p->source_tensor_count) return fail(err, n, "provenance tensor accounting mismatch");
    if (tensor_count != 0u && p->source_tensor_count != tensor_count) {
        return fail(err, n, "provenance source tensor count %u does not match directory count %u",
                    p->source_tensor_count, tensor_count);
    }
    if (p->safetensors_file_count == 0u) return fail(err, n, "provenance safetensors file count must be non-zero");
    const int has = p->json_size != 0u;
    if (has != ((p->flags & UOCR_PROVENANCE_FLAG_JSON_PAYLOAD) != 0u)) {
        return fail(err, n, "provenance JSON flag does not match payload size");
    }
    if (has && (!in_range(p->json_offset, p->json_size, s->size) || p->json_offset < sizeof(*p))) {
        return fail(err, n, "provenance JSON is outside its section");
    }
    if (!has && p->json_offset != 0u) return fail(err, n, "provenance JSON offset set without JSON size");
    return 0;
}

static int q4_family_allowed(uint32_t f) {
    return f == UOCR_TENSOR_FAMILY_MOE_EXPERT || f == UOCR_TENSOR_FAMILY_LM_HEAD || f == UOCR_TENSOR_FAMILY_MOE_SHARED ||
           f == UOCR_TENSOR_FAMILY_LAYER_DENSE_MLP || f == UOCR_TENSOR_FAMILY_TOK_EMBED ||
           f == UOCR_TENSOR_FAMILY_VISION_SAM || f == UOCR_TENSOR_FAMILY_VISION_CLIP ||
           f == UOCR_TENSOR_FAMILY_PROJECTOR;
}

/* per-tensor checks (uocr_model_file.c:534-825) */
static int check_tensor(const uocr_tensor_entry *t, uint32_t i, uint32_t qprofile, const uocr_section_entry *data,
                        uint64_t file_size, char *err, size_t n) {
    const int quant = t->qtype == UOCR_TENSOR_Q8_0 || t->qtype == UOCR_TENSOR_Q4_0;
    if (qprofile == UOCR_QPROFILE_FP16 && t->qtype != UOCR_TENSOR_F16) {
        return fail(err, n, "tensor entry %u has non-fp16 qtype %u", i, t->qtype);
    }
    if (t->qtype != UOCR_TENSOR_F16 && t->qtype != UOCR_TENSOR_Q8_0 &&
        !(t->qtype == UOCR_TENSOR_Q4_0 && qprofile == UOCR_QPROFILE_MIXED_Q4)) {
        return fail(err, n, "tensor entry %u has unsupported qtype %u for %s", i, t->qtype, uocr_qprofile_name(qprofile));
    }
    if (t->rank == 0u || t->rank > UOCR_TENSOR_MAX_DIMS || (quant && t->rank != 2u)) {
        return fail(err, n, "tensor entry %u rank %u is invalid for %s", i, t->rank, uocr_qtype_name(t->qtype));
    }
    uint64_t elems = 1u;
    for (uint32_t d = 0; d < t->rank; ++d) {
        if (t->logical_shape[d] == 0u || t->physical_shape[d] != t->logical_shape[d]) {
            return fail(err, n, "tensor entry %u has a zero or non-logical physical dimension %u", i, d);
        }
        elems *= t->logical_shape[d];
    }
    if (t->qtype == UOCR_TENSOR_F16) {
        if (t->payload_size != elems * 2u) return fail(err, n, "tensor entry %u fp16 payload size mismatch", i);
        if (t->block_size || t->row_size || t->scale_offset || t->scale_size || t->min_offset || t->min_size) {
            return fail(err, n, "tensor entry %u fp16 tensor has non-fp16 packing metadata", i);
        }
        return 0;
    }
    if (t->qtype == UOCR_TENSOR_Q4_0 && !q4_family_allowed(t->family)) {
        return fail(err, n, "tensor entry %u q4_0 is not supported for family %u", i, t->family);
    }
    const uint32_t rows = t->logical_shape[0], cols = t->logical_shape[1];
    if ((t->flags & UOCR_TENSOR_FLAG_ROW_MAJOR) == 0u ||
        (t->flags & (UOCR_TENSOR_FLAG_TRANSPOSED | UOCR_TENSOR_FLAG_FLATTENED_LEADING_DIM)) != 0u) {
        return fail(err, n, "tensor entry %u %s tensor must be row-major and not transformed", i, uocr_qtype_name(t->qtype));
    }
    if (t->block_size != UOCR_QGROUP || cols % UOCR_QGROUP != 0u) {
        return fail(err, n, "tensor entry %u %s block size/cols mismatch", i, uocr_qtype_name(t->qtype));
    }
    const uint32_t row_size = t->qtype == UOCR_TENSOR_Q8_0 ? cols : cols / 2u;
    if (t->row_size != row_size) return fail(err, n, "tensor entry %u row size mismatch: got %u expected %u", i, t->row_size, row_size);
    if (t->payload_size != (uint64_t)rows * row_size) return fail(err, n, "tensor entry %u payload size mismatch", i);
    if (t->scale_size != (uint64_t)rows * (cols / UOCR_QGROUP) * 2u) return fail(err, n, "tensor entry %u scale size mismatch", i);
    if (t->scale_offset % UOCR_TENSOR_PAYLOAD_ALIGNMENT != 0u) return fail(err, n, "tensor entry %u scale offset is not aligned", i);
    if (!in_range(t->scale_offset, t->scale_size, file_size) || !in_section(t->scale_offset, t->scale_size, data)) {
        return fail(err, n, "tensor entry %u scale is outside tensor-data section", i);
    }
    if (t->min_offset != 0u || t->min_size != 0u) return fail(err, n, "tensor entry %u has min metadata", i);
    if (t->qtype_reason != 0u || t->promotion_reason != 0u) return fail(err, n, "tensor entry %u has unknown reasons", i);
    return 0;
}

static int validate(const uint8_t *b, size_t size, uocr_model_file *m, char *err, size_t n) {
    if (b == NULL) return fail(err, n, "model data pointer is null");
    if (size < sizeof(uocr_file_header)) return fail(err, n, "file too small for UOCR header: %zu bytes", size);
    const uocr_file_header *h = (const uocr_file_header *)(const void *)b;
    if (memcmp(h->magic, UOCR_FILE_MAGIC, 4) != 0) return fail(err, n, "bad UOCR magic");
    if (h->version != UOCR_FORMAT_VERSION) return fail(err, n, "unsupported UOCR format version %u", h->version);
    if (h->header_size != sizeof(uocr_file_header)) return fail(err, n, "unexpected UOCR header size %u", h->header_size);
    if (h->endian_marker != UOCR_ENDIAN_MARKER) return fail(err, n, "unsupported endian marker 0x%08x", h->endian_marker);
    if (h->file_size != (uint64_t)size) {
        return fail(err, n, "file_size mismatch: header says %llu, actual is %zu", (unsigned long long)h->file_size, size);
    }
    if (h->required_alignment == 0u) return fail(err, n, "required alignment must be non-zero");
    if (h->qprofile != UOCR_QPROFILE_FP16 && h->qprofile != UOCR_QPROFILE_MIXED_Q8_0 && h->qprofile != UOCR_QPROFILE_MIXED_Q4) {
        return fail(err, n, "unsupported .uocr qprofile %u", h->qprofile);
    }
    if (h->section_count == 0u) return fail(err, n, "section_count must be non-zero");
    const uint64_t dir_bytes = (uint64_t)h->section_count * sizeof(uocr_section_entry);
    if (!in_range(h->section_dir_offset, dir_bytes, size)) return fail(err, n, "section directory is out of range");
    if (h->section_dir_offset % 8u != 0u) return fail(err, n, "section directory offset must be 8-byte aligned");
    const uocr_section_entry *sec = (const uocr_section_entry *)(const void *)(b + h->section_dir_offset);
    for (uint32_t i = 0; i < h->section_count; ++i) {
        const uocr_section_entry *s = &sec[i];
        if (!in_range(s->offset, s->size, size)) return fail(err, n, "section %u is out of range", i);
        if (s->alignment != 0u && s->offset % s->alignment != 0u) return fail(err, n, "section %u offset is not aligned", i);
        if (s->size != 0u) {
            if (s->offset < h->header_size) return fail(err, n, "section %u overlaps file header", i);
            if (s->offset < h->section_dir_offset + dir_bytes && h->section_dir_offset < s->offset + s->size) {
                return fail(err, n, "section %u overlaps section directory", i);
            }
        }
        for (uint32_t j = 0; j < i; ++j) {
            if (sec[j].type == s->type) return fail(err, n, "duplicate section type %u", s->type);
            if (sec[j].size && s->size && sec[j].offset < s->offset + s->size && s->offset < sec[j].offset + sec[j].size) {
                return fail(err, n, "section %u overlaps section %u", i, j);
            }
        }
    }
    const uocr_section_entry *cfg = find_section(h, sec, UOCR_SECTION_CONFIG);
    if (cfg == NULL) return fail(err, n, "missing config section");
    if (cfg->size < sizeof(uocr_config_record)) return fail(err, n, "config section too small");
    const uocr_config_record *config = (const uocr_config_record *)(const void *)(b + cfg->offset);
    if (check_config(config, err, n) != 0) return -1;
    if (check_tokenizer(b, find_section(h, sec, UOCR_SECTION_TOKENIZER_METADATA), err, n) != 0) return -1;

    const uocr_section_entry *dsec = find_section(h, sec, UOCR_SECTION_TENSOR_DIRECTORY);
    const uocr_section_entry *data = find_section(h, sec, UOCR_SECTION_TENSOR_DATA);
    const uocr_tensor_entry *ents = NULL;
    uint32_t count = 0;
    if (dsec != NULL) {
        if (dsec->size < sizeof(uocr_tensor_directory_header)) return fail(err, n, "tensor directory section too small");
        const uocr_tensor_directory_header *dh = (const uocr_tensor_directory_header *)(const void *)(b + dsec->offset);
        if (dh->magic != UOCR_TENSOR_DIR_MAGIC) return fail(err, n, "bad tensor directory magic 0x%08x", dh->magic);
        if (dh->version != UOCR_FORMAT_VERSION) return fail(err, n, "unsupported tensor directory version %u", dh->version);
        if (dh->entry_size != sizeof(uocr_tensor_entry)) return fail(err, n, "unexpected tensor directory entry size %u", dh->entry_size);
        const uint64_t eb = (uint64_t)dh->tensor_count * sizeof(uocr_tensor_entry);
        if (dsec->size != sizeof(*dh) + eb) return fail(err, n, "tensor directory size/count mismatch");
        if (data != NULL && (data->alignment < UOCR_TENSOR_DATA_ALIGNMENT || data->offset % UOCR_TENSOR_DATA_ALIGNMENT != 0u)) {
            return fail(err, n, "tensor-data section is not page aligned");
        }
        ents = (const uocr_tensor_entry *)(const void *)(b + dsec->offset + sizeof(*dh));
        count = dh->tensor_count;
        const uint32_t known = UOCR_TENSOR_FLAG_ROW_MAJOR | UOCR_TENSOR_FLAG_TRANSPOSED | UOCR_TENSOR_FLAG_FLATTENED_LEADING_DIM;
        for (uint32_t i = 0; i < count; ++i) {
            const uocr_tensor_entry *t = &ents[i];
            if (t->id == 0u) return fail(err, n, "tensor entry %u has invalid id 0", i);
            if (i > 0u && ents[i - 1u].id >= t->id) return fail(err, n, "tensor entry %u id %u is not greater than previous id %u", i, t->id, ents[i - 1u].id);
            if (t->rank > UOCR_TENSOR_MAX_DIMS) return fail(err, n, "tensor entry %u rank %u exceeds limit", i, t->rank);
            if ((t->flags & ~known) != 0u) return fail(err, n, "tensor entry %u has unknown flags 0x%x", i, t->flags);
            if ((t->flags & UOCR_TENSOR_FLAG_TRANSPOSED) != 0u) return fail(err, n, "tensor entry %u requests unsupported transposed layout", i);
            if (t->usage == UOCR_TENSOR_USAGE_OMITTED_WITH_REASON) {
                if (t->payload_offset || t->payload_size || t->scale_offset || t->scale_size || t->min_offset || t->min_size) {
                    return fail(err, n, "omitted tensor entry %u has payload bytes", i);
                }
                continue;
            }
            if (t->usage != UOCR_TENSOR_USAGE_RUNTIME && t->usage != UOCR_TENSOR_USAGE_PRESERVED_UNUSED) {
                return fail(err, n, "tensor entry %u has unknown usage %u", i, t->usage);
            }
            if (data == NULL) return fail(err, n, "tensor entry %u has payload but tensor-data section is missing", i);
            if (t->payload_size == 0u) return fail(err, n, "tensor entry %u has zero payload size", i);
            if (t->payload_offset % UOCR_TENSOR_PAYLOAD_ALIGNMENT != 0u) return fail(err, n, "tensor entry %u payload offset is not aligned", i);
            if (check_tensor(t, i, h->qprofile, data, size, err, n) != 0) return -1;
            if (!in_range(t->payload_offset, t->payload_size, size) || !in_section(t->payload_offset, t->payload_size, data)) {
                return fail(err, n, "tensor entry %u payload is outside tensor-data section", i);
            }
        }
    }
    if (check_provenance(b, h, find_section(h, sec, UOCR_SECTION_PROVENANCE), count, err, n) != 0) return -1;
    m->data = b;
    m->size = size;
    m->header = h;
    m->sections = sec;
    m->config = config;
    m->tensors = ents;
    m->tensor_count = count;
    m->tensor_data_bytes = data != NULL ? data->size : 0u;
    return 0;
}

int uocr_model_open_memory(const void *data, size_t size, uocr_model_file *out, char *err, size_t n) {
    if (err != NULL && n > 0u) err[0] = '\0';
    if (out == NULL) return fail(err, n, "output model file pointer is null");
    memset(out, 0, sizeof(*out));
    return validate((const uint8_t *)data, size, out, err, n);
}

int uocr_model_open_path(const char *path, uocr_model_file *out, char *err, size_t n) {
    if (err != NULL && n > 0u) err[0] = '\0';
    if (out == NULL) return fail(err, n, "output model file pointer is null");
    memset(out, 0, sizeof(*out));
    if (path == NULL) return fail(err, n, "path is null");
    FILE *f = fopen(path, "rb");
    if (f == NULL) return fail(err, n, "failed to open '%s': %s", path, strerror(errno));
    if (fseeko(f, 0, SEEK_END) != 0) {
        fclose(f);
        return fail(err, n, "failed to seek '%s'", path);
    }
    const off_t len = ftello(f);
    if (len < 0 || fseeko(f, 0, SEEK_SET) != 0) {
        fclose(f);
        return fail(err, n, "failed to size '%s'", path);
    }
    uint8_t *buf = (uint8_t *)malloc(len > 0 ? (size_t)len : 1u);
    if (buf == NULL) {
        fclose(f);
        return fail(err, n, "failed to allocate %lld bytes", (long long)len);
    }
    if ((size_t)len != 0u && fread(buf, 1, (size_t)len, f) != (size_t)len) {
        free(buf);
        fclose(f);
        return fail(err, n, "failed to read '%s'", path);
    }
    fclose(f);
    if (validate(buf, (size_t)len, out, err, n) != 0) {
        free(buf);
        memset(out, 0, sizeof(*out));
        return -1;
    }
    out->owned = buf;
    return 0;
}

void uocr_model_close(uocr_model_file *m) {
    if (m == NULL) return;
    free(m->owned);
    memset(m, 0, sizeof(*m));
}

const uocr_tensor_entry *uocr_model_find(const uocr_model_file *m, uint32_t id) {
    if (m == NULL || m->tensors == NULL || id == 0u) return NULL;
    uint32_t lo = 0, hi = m->tensor_count;
    while (lo < hi) {
        const uint32_t mid = lo + (hi - lo) / 2u;
        if (m->tensors[mid].id == id) return &m->tensors[mid];
        if (m->tensors[mid].id < id) lo = mid + 1u; else hi = mid;
    }
    return NULL;
}

/* ---- binding (uocr_metal.m:2728-2763 allow-lists) ----------------------- */

enum { ALLOW_F16 = 1, ALLOW_Q8 = 2, ALLOW_Q4 = 4 };

static int bind_one(const uocr_model_file *m, uint32_t id, uint32_t rank, uint32_t rows, uint32_t cols, int allow,
                    const char *what, uocr_bound_tensor *t, uint64_t *total, char *err, size_t n) {
    const uocr_tensor_entry *e = uocr_model_find(m, id);
    if (e == NULL) return fail(err, n, "missing decoder tensor %u (%s)", id, what);
    if (e->usage != UOCR_TENSOR_USAGE_RUNTIME) return fail(err, n, "decoder tensor %u (%s) is not a runtime tensor", id, what);
    const uint32_t r = rank == 1u ? 1u : e->logical_shape[0];
    const uint32_t c = rank == 1u ? e->logical_shape[0] : e->logical_shape[1];
    if (e->rank != rank || r != rows || c != cols) {
        return fail(err, n, "decoder tensor %u (%s) shape mismatch: expected [%u,%u]", id, what, rows, cols);
    }
    const int bit = e->qtype == UOCR_TENSOR_F16 ? ALLOW_F16 : e->qtype == UOCR_TENSOR_Q8_0 ? ALLOW_Q8
                    : e->qtype == UOCR_TENSOR_Q4_0 ? ALLOW_Q4 : 0;
    if ((allow & bit) == 0) {
        return fail(err, n, "decoder tensor %u (%s) qtype %s is not allowed for this role", id, what, uocr_qtype_name(e->qtype));
    }
    t->qtype = e->qtype;
    t->rows = rows;
    t->cols = cols;
    t->w = m->data + e->payload_offset;
    t->w_bytes = e->payload_size;
    t->s = e->scale_size != 0u ? m->data + e->scale_offset : NULL;
    t->s_bytes = e->scale_size;
    *total += t->w_bytes + t->s_bytes;
    return 0;
}

int uocr_bind_decoder(const uocr_model_file *m, uocr_decoder_bindings *b, char *err, size_t n) {
    if (m == NULL || b == NULL || m->tensors == NULL) return fail(err, n, "model has no tensor directory");
    memset(b, 0, sizeof(*b));
    const uint32_t H = UOCR_HIDDEN_SIZE, V = UOCR_VOCAB_SIZE;
    const int W_ANY = ALLOW_F16 | ALLOW_Q8 | ALLOW_Q4;
    uint64_t *tot = &b->total_bytes;
    if (bind_one(m, UOCR_TID_TOK_EMBED, 2, V, H, W_ANY, "token embedding", &b->embed, tot, err, n) ||
        bind_one(m, UOCR_TID_LM_HEAD, 2, V, H, W_ANY, "lm head", &b->lm_head, tot, err, n) ||
        bind_one(m, UOCR_TID_FINAL_NORM, 1, 1, H, ALLOW_F16, "final norm", &b->final_norm, tot, err, n)) {
        return -1;
    }
    for (uint32_t l = 0; l < UOCR_DECODER_LAYERS; ++l) {
        uocr_bound_layer *L = &b->layers[l];
        if (bind_one(m, uocr_tid_layer(l, UOCR_TID_L_INPUT_NORM), 1, 1, H, ALLOW_F16, "input norm", &L->in_norm, tot, err, n) ||
            bind_one(m, uocr_tid_layer(l, UOCR_TID_L_POST_ATTN_NORM), 1, 1, H, ALLOW_F16, "post-attention norm", &L->post_norm, tot, err, n) ||
            bind_one(m, uocr_tid_layer(l, UOCR_TID_L_ATTN_Q), 2, H, H, ALLOW_F16 | ALLOW_Q8, "q_proj", &L->q, tot, err, n) ||
            bind_one(m, uocr_tid_layer(l, UOCR_TID_L_ATTN_K), 2, H, H, ALLOW_F16 | ALLOW_Q8, "k_proj", &L->k, tot, err, n) ||
            bind_one(m, uocr_tid_layer(l, UOCR_TID_L_ATTN_V), 2, H, H, ALLOW_F16 | ALLOW_Q8, "v_proj", &L->v, tot, err, n) ||
            bind_one(m, uocr_tid_layer(l, UOCR_TID_L_ATTN_O), 2, H, H, ALLOW_F16 | ALLOW_Q8, "o_proj", &L->o, tot, err, n)) {
            return -1;
        }
        if (L->q.qtype != L->k.qtype || L->q.qtype != L->v.qtype) {
            return fail(err, n, "layer %u q/k/v projections must share one qtype", l);
        }
        if (l == 0u) {
            const uint32_t I = UOCR_DENSE_LAYER0_INTERMEDIATE;
            if (bind_one(m, uocr_tid_layer(0, UOCR_TID_L_DENSE_GATE), 2, I, H, W_ANY, "dense gate", &L->gate, tot, err, n) ||
                bind_one(m, uocr_tid_layer(0, UOCR_TID_L_DENSE_UP), 2, I, H, W_ANY, "dense up", &L->up, tot, err, n) ||
                bind_one(m, uocr_tid_layer(0, UOCR_TID_L_DENSE_DOWN), 2, H, I, W_ANY, "dense down", &L->down, tot, err, n)) {
                return -1;
            }
            if (L->gate.qtype != L->up.qtype) return fail(err, n, "dense gate/up must share one qtype");
            continue;
        }
        const uint32_t SI = UOCR_MOE_SHARED_INTERMEDIATE, EI = UOCR_MOE_EXPERT_INTERMEDIATE;
        if (bind_one(m, uocr_tid_layer(l, UOCR_TID_L_MOE_ROUTER), 2, UOCR_ROUTED_EXPERTS, H, ALLOW_F16, "router", &L->router, tot, err, n) ||
            bind_one(m, uocr_tid_layer(l, UOCR_TID_L_SHARED_GATE), 2, SI, H, W_ANY, "shared gate", &L->sgate, tot, err, n) ||
            bind_one(m, uocr_tid_layer(l, UOCR_TID_L_SHARED_UP), 2, SI, H, W_ANY, "shared up", &L->sup, tot, err, n) ||
            bind_one(m, uocr_tid_layer(l, UOCR_TID_L_SHARED_DOWN), 2, H, SI, W_ANY, "shared down", &L->sdown, tot, err, n)) {
            return -1;
        }
        if (L->sgate.qtype != L->sup.qtype) return fail(err, n, "layer %u shared gate/up must share one qtype", l);
        for (uint32_t e = 0; e < UOCR_ROUTED_EXPERTS; ++e) {
            if (bind_one(m, uocr_tid_expert(l, e, 0), 2, EI, H, W_ANY, "expert gate", &L->egate[e], tot, err, n) ||
                bind_one(m, uocr_tid_expert(l, e, 1), 2, EI, H, W_ANY, "expert up", &L->eup[e], tot, err, n) ||
                bind_one(m, uocr_tid_expert(l, e, 2), 2, H, EI, W_ANY, "expert down", &L->edown[e], tot, err, n)) {
                return -1;
            }
            if (L->egate[e].qtype != L->egate[0].qtype || L->eup[e].qtype != L->egate[0].qtype ||
                L->edown[e].qtype != L->edown[0].qtype) {
                return fail(err, n, "layer %u routed experts must share one qtype per projection", l);
            }
        }
    }
    return 0;
}
