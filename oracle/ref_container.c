/* ref_container.c - test-only probe of QStream's own QSF container reader.
 *
 * Test infrastructure, never part of the product.  Linked with the
 * reference's src/format.c, src/file_access.c and src/error.c and compiled
 * against its include/qsf headers (oracle/Makefile), it lets the tests run
 * the reference's qsf_model_load (src/format.c:99-201) and
 * qsf_decompress_layer (src/format.c:217-288) on files this build writes,
 * and read the on-disk structs' layout (include/qsf/types.h:185-312) as the
 * reference's own compiler lays them out.
 */
#include "qsf/format.h"

#include <stddef.h>
#include <stdint.h>
#include <string.h>

/* What one qsf_model_load call saw. */
typedef struct {
    int32_t  rc;                  /* QSFError */
    uint32_t head_dim, num_kv_heads;
    int32_t  is_gated_ffn, uses_rope, uses_alibi;
    int32_t  has_bias_attn_qkv, has_bias_attn_o, has_bias_ffn, has_bias_norm, weight_tied;
    uint64_t file_size;
    uint8_t  header[256];         /* model->header as loaded */
} ref_summary;

/* qsf_model_load(path, mmap) into *out; the first max_layers layer-index
 * entries (48 bytes each) into layer_index, and for each layer the file
 * offset of the data qsf_decompress_layer returns (-1 when NULL).  Returns
 * the QSFError. */
int ref_container_load(const char* path, ref_summary* out, uint8_t* layer_index, uint32_t max_layers,
                       int64_t* layer_data_off) {
    QSFModel m;
    memset(out, 0, sizeof *out);
    QSFError e = qsf_model_load(&m, path, 1);
    out->rc = (int32_t)e;
    if (e != QSF_OK) return (int)e;
    memcpy(out->header, &m.header, sizeof out->header);
    out->head_dim = m.head_dim;
    out->num_kv_heads = m.num_kv_heads;
    out->is_gated_ffn = m.is_gated_ffn;
    out->uses_rope = m.uses_rope;
    out->uses_alibi = m.uses_alibi;
    out->has_bias_attn_qkv = m.has_bias_attn_qkv;
    out->has_bias_attn_o = m.has_bias_attn_o;
    out->has_bias_ffn = m.has_bias_ffn;
    out->has_bias_norm = m.has_bias_norm;
    out->weight_tied = m.weight_tied;
    out->file_size = m.file.file_size;
    const uint32_t n = m.header.num_layers < max_layers ? m.header.num_layers : max_layers;
    memcpy(layer_index, m.layer_index, (size_t)n * sizeof(QSFLayerIndex));
    for (uint32_t i = 0; i < n; i++) {
        const void* p = qsf_decompress_layer(&m, i, NULL, 0);
        layer_data_off[i] = p && m.file.mmap_ptr ? (int64_t)((const uint8_t*)p - (const uint8_t*)m.file.mmap_ptr)
                                                 : -1;
    }
    qsf_model_free(&m);
    return 0;
}

const char* ref_container_error(void) { return qsf_get_error_detail(); }

/* sizeof and offsetof of every on-disk struct field, by name */
#define SZ(T) {#T, (long)sizeof(T)}
#define OF(T, f) {#T "." #f, (long)offsetof(T, f)}
static const struct {
    const char* name;
    long value;
} k_layout[] = {
    SZ(QSFHeader), OF(QSFHeader, magic), OF(QSFHeader, version), OF(QSFHeader, header_size),
    OF(QSFHeader, arch), OF(QSFHeader, num_layers), OF(QSFHeader, hidden_dim), OF(QSFHeader, num_heads),
    OF(QSFHeader, num_kv_heads), OF(QSFHeader, vocab_size), OF(QSFHeader, max_seq_len),
    OF(QSFHeader, intermediate_dim), OF(QSFHeader, head_dim), OF(QSFHeader, quant_type),
    OF(QSFHeader, activation), OF(QSFHeader, norm_type), OF(QSFHeader, pos_enc_type),
    OF(QSFHeader, rope_theta), OF(QSFHeader, norm_epsilon), OF(QSFHeader, block_size),
    OF(QSFHeader, layer_index_offset), OF(QSFHeader, embedding_offset), OF(QSFHeader, final_offset),
    OF(QSFHeader, tokenizer_offset), OF(QSFHeader, extended_config_offset),
    OF(QSFHeader, calibration_offset), OF(QSFHeader, importance_offset), OF(QSFHeader, bos_token_id),
    OF(QSFHeader, eos_token_id), OF(QSFHeader, pad_token_id), OF(QSFHeader, unk_token_id),
    OF(QSFHeader, num_params_millions), OF(QSFHeader, has_bias), OF(QSFHeader, ffn_type),
    OF(QSFHeader, attn_type), OF(QSFHeader, weight_tying), OF(QSFHeader, rope_scaling_type),
    OF(QSFHeader, rope_scaling_factor), OF(QSFHeader, sliding_window), OF(QSFHeader, tie_word_embeddings),
    OF(QSFHeader, total_file_size), OF(QSFHeader, header_crc32), OF(QSFHeader, endian_marker),
    OF(QSFHeader, num_experts), OF(QSFHeader, num_active_experts), OF(QSFHeader, moe_norm_topk),
    OF(QSFHeader, reserved_moe), OF(QSFHeader, expert_intermediate_dim), OF(QSFHeader, reserved),
    SZ(QSFLayerIndex), OF(QSFLayerIndex, offset), OF(QSFLayerIndex, compressed_size),
    OF(QSFLayerIndex, decompressed_size), OF(QSFLayerIndex, quant_type), OF(QSFLayerIndex, compression_type),
    OF(QSFLayerIndex, num_tensors), OF(QSFLayerIndex, crc32_compressed), OF(QSFLayerIndex, crc32_decompressed),
    OF(QSFLayerIndex, importance_score), OF(QSFLayerIndex, weight_bytes), OF(QSFLayerIndex, layer_ffn_dim),
    OF(QSFLayerIndex, reserved),
    SZ(QSFTensorHeader), OF(QSFTensorHeader, tensor_type), OF(QSFTensorHeader, quant_type),
    OF(QSFTensorHeader, data_layout), OF(QSFTensorHeader, rows), OF(QSFTensorHeader, cols),
    OF(QSFTensorHeader, data_size), OF(QSFTensorHeader, num_outliers), OF(QSFTensorHeader, reserved),
    SZ(QSFEmbeddingHeader), OF(QSFEmbeddingHeader, quant_type), OF(QSFEmbeddingHeader, compressed_size),
    OF(QSFEmbeddingHeader, num_vectors), OF(QSFEmbeddingHeader, embedding_dim),
    OF(QSFEmbeddingHeader, compression_type), OF(QSFEmbeddingHeader, reserved1), OF(QSFEmbeddingHeader, crc32),
    OF(QSFEmbeddingHeader, num_chunks), OF(QSFEmbeddingHeader, chunk_size),
    SZ(QSFFinalHeader), OF(QSFFinalHeader, output_head_type), OF(QSFFinalHeader, final_norm_size),
    OF(QSFFinalHeader, output_head_size), OF(QSFFinalHeader, crc32),
    SZ(QSFOutlierEntry), OF(QSFOutlierEntry, flat_index), OF(QSFOutlierEntry, fp16_value),
};

int ref_layout_count(void) { return (int)(sizeof k_layout / sizeof k_layout[0]); }
const char* ref_layout_name(int i) { return i >= 0 && i < ref_layout_count() ? k_layout[i].name : NULL; }
long ref_layout_value(int i) { return i >= 0 && i < ref_layout_count() ? k_layout[i].value : -1; }
