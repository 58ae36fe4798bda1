/*
 * uocr_format.h - on-disk .uocr model-file format and model constants.
 *
 * The byte layout is the reference's format (src/model/uocr_format.h:8-313,
 * constants src/model/uocr_constants.h:6-93, tensor ids
 * src/model/uocr_tensor_registry.h:11-124): a file written by the reference
 * converter (src/unlimitedocr_c/convert.py:2528) must load here unchanged,
 * so every packed struct keeps the reference field order and size.
 */
#ifndef UOCR_FORMAT_H
#define UOCR_FORMAT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- model constants (uocr_constants.h:6-93) ---------------------------- */
#define UOCR_VOCAB_SIZE 129280u
#define UOCR_BPE_VOCAB_SIZE 128000u
#define UOCR_ADDED_TOKEN_COUNT 830u
#define UOCR_TOKEN_BOS 0
#define UOCR_TOKEN_EOS 1
#define UOCR_TOKEN_PAD 2
#define UOCR_TOKEN_IMAGE 128815
#define UOCR_HIDDEN_SIZE 1280u
#define UOCR_DECODER_LAYERS 12u
#define UOCR_ATTENTION_HEADS 10u
#define UOCR_KV_HEADS 10u
#define UOCR_HEAD_DIM 128u
#define UOCR_ROPE_THETA 10000u
#define UOCR_RMS_NORM_EPS 1.0e-6f
#define UOCR_MAX_POSITIONS 32768u
#define UOCR_GENERATED_RING_WINDOW 128u
#define UOCR_DENSE_FIRST_LAYERS 1u
#define UOCR_ROUTED_EXPERTS 64u
#define UOCR_MOE_TOP_K 6u
#define UOCR_MOE_EXPERT_INTERMEDIATE 896u
#define UOCR_MOE_SHARED_EXPERTS 2u
#define UOCR_MOE_SHARED_INTERMEDIATE 1792u
#define UOCR_DENSE_LAYER0_INTERMEDIATE 6848u
#define UOCR_MOE_ROUTED_SCALING_FACTOR 1.0f
#define UOCR_MOE_NORM_TOPK_PROB 0u
#define UOCR_PROJECTOR_IN_SIZE 2048u
#define UOCR_VISION_PATCH_SIZE 16u
#define UOCR_DOWNSAMPLE_RATIO 4u
#define UOCR_GLOBAL_VIEW_SIZE 1024u
#define UOCR_LOCAL_VIEW_SIZE 640u
#define UOCR_DEFAULT_MAX_BATCH 1u
#define UOCR_DEFAULT_MAX_PROMPT_TOKENS 4096u
#define UOCR_DEFAULT_MAX_GEN_TOKENS 512u

/* ---- file layout (uocr_format.h:8-13) ---------------------------------- */
#define UOCR_FILE_MAGIC "UOCR"
#define UOCR_FORMAT_VERSION 1u
#define UOCR_ENDIAN_MARKER 0x01020304u
#define UOCR_FILE_ALIGNMENT 4096u
#define UOCR_TENSOR_DATA_ALIGNMENT 4096u
#define UOCR_TENSOR_PAYLOAD_ALIGNMENT 16u

enum {
    UOCR_QPROFILE_FP16 = 1,
    UOCR_QPROFILE_MIXED_Q8_0 = 2,
    UOCR_QPROFILE_MIXED_Q4 = 3
};

enum {
    UOCR_SECTION_CONFIG = 1,
    UOCR_SECTION_TENSOR_DIRECTORY = 2,
    UOCR_SECTION_TOKENIZER_METADATA = 3,
    UOCR_SECTION_PROVENANCE = 4,
    UOCR_SECTION_TENSOR_DATA = 5
};

#define UOCR_TOKENIZER_FLAG_C_V1_NOT_REQUIRED (1u << 0)
#define UOCR_TOKENIZER_FLAG_EMBEDDED_PAYLOAD (1u << 1)
#define UOCR_PROVENANCE_FLAG_JSON_PAYLOAD (1u << 0)

enum {
    UOCR_TENSOR_F16 = 1,
    UOCR_TENSOR_F32 = 2,
    UOCR_TENSOR_Q8_0 = 3,
    UOCR_TENSOR_Q4_0 = 4,
    UOCR_TENSOR_Q4_1 = 5
};

/* Q8_0: int8 q in [-127,127], row-major [rows][cols], one fp16 scale per 64
 * columns in a separate [rows][cols/64] region.  w = q * scale.
 * Q4_0: nibble = q + 8 with q in [-8,7]; byte j (0..31) of each 64-column
 * group holds column j in its low nibble and column j+32 in its high nibble;
 * fp16 scale per group (may be negative).  w = (nibble - 8) * scale. */
#define UOCR_QGROUP 64u
#define UOCR_Q8_MIN (-127)
#define UOCR_Q8_MAX 127
#define UOCR_Q4_MIN (-8)
#define UOCR_Q4_MAX 7

enum {
    UOCR_TENSOR_USAGE_RUNTIME = 1,
    UOCR_TENSOR_USAGE_PRESERVED_UNUSED = 2,
    UOCR_TENSOR_USAGE_OMITTED_WITH_REASON = 3
};

#define UOCR_TENSOR_FLAG_ROW_MAJOR (1u << 0)
#define UOCR_TENSOR_FLAG_TRANSPOSED (1u << 1)
#define UOCR_TENSOR_FLAG_FLATTENED_LEADING_DIM (1u << 2)

enum {
    UOCR_TENSOR_FAMILY_UNKNOWN = 0,
    UOCR_TENSOR_FAMILY_TOK_EMBED = 1,
    UOCR_TENSOR_FAMILY_LM_HEAD = 2,
    UOCR_TENSOR_FAMILY_FINAL_NORM = 3,
    UOCR_TENSOR_FAMILY_LAYER_ATTN = 4,
    UOCR_TENSOR_FAMILY_LAYER_NORM = 5,
    UOCR_TENSOR_FAMILY_LAYER_DENSE_MLP = 6,
    UOCR_TENSOR_FAMILY_MOE_ROUTER = 7,
    UOCR_TENSOR_FAMILY_MOE_EXPERT = 8,
    UOCR_TENSOR_FAMILY_MOE_SHARED = 9,
    UOCR_TENSOR_FAMILY_VISION_SAM = 10,
    UOCR_TENSOR_FAMILY_VISION_CLIP = 11,
    UOCR_TENSOR_FAMILY_PROJECTOR = 12,
    UOCR_TENSOR_FAMILY_IMAGE_NEWLINE = 13,
    UOCR_TENSOR_FAMILY_VIEW_SEPARATOR = 14
};

enum {
    UOCR_TENSOR_PROJ_NONE = 0,
    UOCR_TENSOR_PROJ_WEIGHT = 1,
    UOCR_TENSOR_PROJ_BIAS = 2,
    UOCR_TENSOR_PROJ_Q = 10,
    UOCR_TENSOR_PROJ_K = 11,
    UOCR_TENSOR_PROJ_V = 12,
    UOCR_TENSOR_PROJ_O = 13,
    UOCR_TENSOR_PROJ_GATE = 20,
    UOCR_TENSOR_PROJ_UP = 21,
    UOCR_TENSOR_PROJ_DOWN = 22
};

#define UOCR_TOKENIZER_METADATA_MAGIC 0x4b4f5455u /* "UTOK" */
#define UOCR_PROVENANCE_MAGIC 0x564f5250u         /* "PROV" */
#define UOCR_TENSOR_DIR_MAGIC 0x52494454u         /* "TDIR" */
#define UOCR_TENSOR_MAX_DIMS 4u

#define UOCR_PACKED __attribute__((packed))

typedef struct UOCR_PACKED uocr_file_header {
    char magic[4];
    uint32_t version;
    uint32_t header_size;
    uint32_t endian_marker;
    uint32_t required_alignment;
    uint32_t qprofile;
    uint32_t section_count;
    uint32_t reserved0;
    uint64_t file_size;
    uint64_t section_dir_offset;
    uint8_t model_id_hash[32];
    uint8_t reserved1[32];
} uocr_file_header;

typedef struct UOCR_PACKED uocr_section_entry {
    uint32_t type;
    uint32_t flags;
    uint64_t offset;
    uint64_t size;
    uint64_t alignment;
} uocr_section_entry;

typedef struct UOCR_PACKED uocr_config_record {
    uint32_t vocab_size;
    uint32_t bpe_vocab_size;
    uint32_t added_token_count;
    uint32_t bos_token_id;
    uint32_t eos_token_id;
    uint32_t pad_token_id;
    uint32_t image_token_id;
    uint32_t hidden_size;
    uint32_t decoder_layers;
    uint32_t attention_heads;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t rope_theta;
    uint32_t max_positions;
    uint32_t generated_ring_window;
    uint32_t dense_first_layers;
    uint32_t routed_experts;
    uint32_t moe_top_k;
    uint32_t moe_expert_intermediate;
    uint32_t shared_experts;
    uint32_t dense_layer0_intermediate;
    uint32_t projector_in;
    uint32_t projector_out;
    uint32_t vision_patch_size;
    uint32_t downsample_ratio;
    uint32_t supported_global_view;
    uint32_t supported_local_view;
} uocr_config_record;

typedef struct UOCR_PACKED uocr_tokenizer_metadata_record {
    uint32_t magic;
    uint32_t version;
    uint32_t record_size;
    uint32_t flags;
    uint8_t tokenizer_hash[32];
    uint32_t vocab_size;
    uint32_t bpe_vocab_size;
    uint32_t added_token_count;
    uint32_t bos_token_id;
    uint32_t eos_token_id;
    uint32_t pad_token_id;
    uint32_t image_token_id;
    uint64_t tokenizer_json_offset;
    uint64_t tokenizer_json_size;
} uocr_tokenizer_metadata_record;

typedef struct UOCR_PACKED uocr_provenance_record {
    uint32_t magic;
    uint32_t version;
    uint32_t record_size;
    uint32_t flags;
    uint32_t source_tensor_count;
    uint32_t runtime_tensor_count;
    uint32_t preserved_unused_tensor_count;
    uint32_t omitted_tensor_count;
    uint32_t safetensors_file_count;
    uint32_t qprofile;
    uint32_t converter_version_major;
    uint32_t converter_version_minor;
    uint32_t converter_version_patch;
    uint32_t reserved0;
    uint8_t config_hash[32];
    uint8_t tokenizer_hash[32];
    uint8_t safetensors_index_hash[32];
    uint8_t reserved_hash[32];
    uint64_t json_offset;
    uint64_t json_size;
} uocr_provenance_record;

typedef struct UOCR_PACKED uocr_tensor_directory_header {
    uint32_t magic;
    uint32_t version;
    uint32_t entry_size;
    uint32_t tensor_count;
} uocr_tensor_directory_header;

typedef struct UOCR_PACKED uocr_tensor_entry {
    uint32_t id;
    uint32_t family;
    int32_t layer;
    int32_t expert;
    uint32_t projection;
    uint32_t usage;
    uint32_t qtype;
    uint32_t flags;
    uint32_t rank;
    uint32_t logical_shape[UOCR_TENSOR_MAX_DIMS];
    uint32_t physical_shape[UOCR_TENSOR_MAX_DIMS];
    uint64_t payload_offset;
    uint64_t payload_size;
    uint32_t block_size;
    uint32_t row_size;
    uint64_t scale_offset;
    uint64_t scale_size;
    uint64_t min_offset;
    uint64_t min_size;
    uint32_t qtype_reason;
    uint32_t promotion_reason;
    uint32_t source_name_offset;
    uint32_t source_name_size;
} uocr_tensor_entry;

#if !defined(__cplusplus)
_Static_assert(sizeof(uocr_file_header) == 112u, "uocr_file_header size");
_Static_assert(sizeof(uocr_section_entry) == 32u, "uocr_section_entry size");
_Static_assert(sizeof(uocr_config_record) == 108u, "uocr_config_record size");
_Static_assert(sizeof(uocr_tokenizer_metadata_record) == 92u, "tokenizer record size");
_Static_assert(sizeof(uocr_provenance_record) == 200u, "provenance record size");
_Static_assert(sizeof(uocr_tensor_directory_header) == 16u, "tensor dir header size");
_Static_assert(sizeof(uocr_tensor_entry) == 140u, "uocr_tensor_entry size");
#endif

/* ---- tensor ids (uocr_tensor_registry.h:11-124) ------------------------ */
#define UOCR_TID_TOK_EMBED 1u
#define UOCR_TID_LM_HEAD 2u
#define UOCR_TID_FINAL_NORM 3u
#define UOCR_TID_LAYER_BASE 10000u
#define UOCR_TID_LAYER_STRIDE 1000u
#define UOCR_TID_L_INPUT_NORM 1u
#define UOCR_TID_L_POST_ATTN_NORM 2u
#define UOCR_TID_L_ATTN_Q 10u
#define UOCR_TID_L_ATTN_K 11u
#define UOCR_TID_L_ATTN_V 12u
#define UOCR_TID_L_ATTN_O 13u
#define UOCR_TID_L_DENSE_GATE 30u
#define UOCR_TID_L_DENSE_UP 31u
#define UOCR_TID_L_DENSE_DOWN 32u
#define UOCR_TID_L_MOE_ROUTER 40u
#define UOCR_TID_L_SHARED_GATE 50u
#define UOCR_TID_L_SHARED_UP 51u
#define UOCR_TID_L_SHARED_DOWN 52u
#define UOCR_TID_L_EXPERT_BASE 100u
#define UOCR_TID_L_EXPERT_STRIDE 3u

static inline uint32_t uocr_tid_layer(uint32_t layer, uint32_t local) {
    return UOCR_TID_LAYER_BASE + layer * UOCR_TID_LAYER_STRIDE + local;
}

/* proj_index: 0 = gate, 1 = up, 2 = down */
static inline uint32_t uocr_tid_expert(uint32_t layer, uint32_t expert, uint32_t proj_index) {
    return uocr_tid_layer(layer, UOCR_TID_L_EXPERT_BASE + expert * UOCR_TID_L_EXPERT_STRIDE + proj_index);
}

#ifdef __cplusplus
}
#endif

#endif /* UOCR_FORMAT_H */
