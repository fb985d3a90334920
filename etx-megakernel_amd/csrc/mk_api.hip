// Host side of the etxmk C ABI (include/etxmk.h): arena layout, seeded initialisation, launches.
//
// Reference counterparts: etx_host (etx/runtime/include/etx/host.h:22-692) for setup / run / wait, and the model
// hosts examples/llm/host.hip:57-244 and examples/vllm_llm/host.hip:126-1159 for buffers and per-step parameters.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <chrono>
#include <initializer_list>
#include <mutex>
#include <thread>
#include <vector>

#include "etxmk.h"
#include "mk_init.h"
#include "mk_mla.h"

namespace mk {
// the persistent kernels live in their own translation units (mk_fused_*.hip, mk_batch_*.hip)
MK_FUSED_SHAPES_BF16(MK_FUSED_DECL)
MK_FUSED_SHAPES_FP8(MK_FUSED_DECL)
MK_BATCH_SHAPES_BF16(MK_BATCH_DECL)
MK_BATCH_SHAPES_FP8(MK_BATCH_DECL)
MK_DS_SHAPES(MK_DS_DECL)

// unfused mode (bf16 weights)
MK_PHASE_KERNEL(etxmk_p_qkv, phase_qkv_any(p, layer, s, NoWait{}))
MK_PHASE_KERNEL(etxmk_p_attn, phase_attn<1>(p, layer, s, NoWait{}))
MK_PHASE_KERNEL(etxmk_p_oproj, phase_oproj_any(p, layer, s, NoWait{}))
MK_PHASE_KERNEL(etxmk_p_router, phase_router_any(p, layer, s, NoWait{}))
MK_PHASE_KERNEL(etxmk_p_expert_up, phase_expert_up_any(p, layer, s, NoWait{}))
MK_PHASE_KERNEL(etxmk_p_expert_down, phase_expert_down_any(p, layer, s, NoWait{}))
MK_PHASE_KERNEL(etxmk_p_gateup, phase_gateup_any(p, layer, s, NoWait{}))
MK_PHASE_KERNEL(etxmk_p_down, phase_down_any(p, layer, s, NoWait{}))
MK_PHASE_KERNEL(etxmk_p_head, phase_head_any(p, s, NoWait{}))
MK_PHASE_KERNEL(etxmk_p_token, phase_token(p, NoWait{}))
}  // namespace mk

using namespace mk;

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

#define HIPCHK(call)                                                                       \
  do {                                                                                     \
    hipError_t e_ = (call);                                                                \
    if (e_ != hipSuccess) return fail(ETXMK_EHIP, "%s: %s", #call, hipGetErrorString(e_)); \
  } while (0)

constexpr uint64_t ALIGN = 256;
constexpr uint64_t SPIN_TICKS_DEFAULT = 200000000ull;   // 2 s of the 100 MHz s_memrealtime clock
inline uint64_t align_up(uint64_t v) { return (v + ALIGN - 1) & ~(ALIGN - 1); }

struct TensorSlot {
  int kind, layer;
  int count;                 // tensors of this shape back to back (experts)
  int rows, cols, perm;      // perm: rows stored lane-permuted
  int fp8;                   // rows in Fp8Row format (codes + scale, cols + 16 bytes) instead of bf16
  uint64_t off;              // byte offset of tensor 0
  int lcols = 0;             // logical row length when the stored rows are padded (0: cols)
  int split = 0;             // DeepSeek-V2 kv_b_proj: stored as W_UK^T then W_UV (etxmk_pack_kvb)
  int logical_cols() const { return lcols ? lcols : cols; }
  uint64_t row_bytes() const { return fp8 ? (uint64_t)cols + 16 : 2ull * cols; }
  uint64_t tensor_bytes() const { return (uint64_t)rows * row_bytes(); }
};

// the matrices held as fp8 when the weight type is ETXMK_W_FP8
bool fp8_kind(int kind) {
  return kind == ETXMK_T_WQKV || kind == ETXMK_T_WO || kind == ETXMK_T_W13 || kind == ETXMK_T_W2 ||
         kind == ETXMK_T_WGU || kind == ETXMK_T_WD;
}

inline uint64_t stream_id(int kind, int layer, int expert) {
  return ((uint64_t)kind << 48) | ((uint64_t)(layer + 1) << 24) | (uint64_t)expert;
}

// row lengths each GEMV phase is instantiated for (MK_K_* in mk_device.h)
bool k_in(int k, std::initializer_list<int> ks) {
  for (int v : ks)
    if (k == v) return true;
  return false;
}

bool is_ds(const etxmk_config& c) { return c.arch == ETXMK_ARCH_DSV2; }
// DeepSeek-V2 derived sizes: fused q_proj + kv_a rows, shared width, dense width rounded up to whole 512 blocks
int ds_nqa(const etxmk_config& c) { return c.NH * (c.qk_nope + c.qk_rope) + c.kv_lora + c.qk_rope; }
int ds_si(const etxmk_config& c) { return c.n_shared * c.MI; }
int ds_ip(const etxmk_config& c) { return (c.dense_I + 511) / 512 * 512; }
int ds_nhg(const etxmk_config& c) { return c.NH < MLA_G ? 1 : c.NH / MLA_G; }
// rows of the fused QKV matrix
int nqkv_of(const etxmk_config& c) { return is_ds(c) ? ds_nqa(c) : (c.NH + 2 * c.NKV) * c.HD; }

// the DeepSeek-V2 persistent kernel for this shape, or nullptr
const void* ds_kernel(const etxmk_config& c) {
#define MK_PICK_DS(name, h_, ka_, km_, ksh_, e_, ip_, b_)                                                          \
  if (c.H == h_ && c.NH * c.v_head == ka_ && c.MI == km_ && ds_si(c) == ksh_ && c.E == e_ &&                     \
      (c.first_dense == 0 || ds_ip(c) == ip_) && c.batch <= b_)                                                   \
    return (const void*)name;
  MK_DS_SHAPES(MK_PICK_DS)
#undef MK_PICK_DS
  return nullptr;
}

// the single-sequence persistent kernel instantiated for this shape and weight type, or nullptr
const void* fused_kernel(const etxmk_config& c) {
  const int km = c.moe ? c.MI : c.I;
#define MK_PICK(name, h_, ka_, km_, moe_, e_, fp8_)                                                               \
  if (c.H == h_ && c.NH * c.HD == ka_ && km == km_ && (c.moe != 0) == moe_ && (!moe_ || c.E == e_) &&            \
      (c.wdtype == ETXMK_W_FP8) == fp8_)                                                                          \
    return (const void*)name;
  MK_FUSED_SHAPES_BF16(MK_PICK)
  MK_FUSED_SHAPES_FP8(MK_PICK)
#undef MK_PICK
  return nullptr;
}

// the batched persistent kernel for this shape and weight type with the smallest batch capacity that holds
// `rows` rows (default c.batch), or nullptr
const void* batch_kernel(const etxmk_config& c, int rows = 0) {
  if (rows <= 0) rows = c.batch;
  const int km = c.moe ? c.MI : c.I;
  const void* best = nullptr;
  int cap = 0;
#define MK_PICK_B(name, h_, ka_, km_, moe_, e_, fp8_, b_)                                                         \
  if (c.H == h_ && c.NH * c.HD == ka_ && km == km_ && (c.moe != 0) == moe_ && (!moe_ || c.E == e_) &&            \
      (c.wdtype == ETXMK_W_FP8) == fp8_ && rows <= b_ && (!best || b_ < cap)) {                                   \
    best = (const void*)name;                                                                                     \
    cap = b_;                                                                                                     \
  }
  MK_BATCH_SHAPES_BF16(MK_PICK_B)
  MK_BATCH_SHAPES_FP8(MK_PICK_B)
#undef MK_PICK_B
  return best;
}

// DeepSeek-V2 (multi-head latent attention): the kernel is built for DeepSeek-V2's head dimensions, bf16 weights,
// block sizes whose 16-position groups share a block, and up to MAX_B_DS sequences
int check_ds(const etxmk_config* c) {
  if (c->kv_lora != MLA_KVL || c->qk_nope != MLA_NOPE || c->qk_rope != MLA_R || c->v_head != MLA_VH)
    return fail(ETXMK_EINVAL, "MLA dims (kv_lora %d, qk_nope %d, qk_rope %d, v_head %d) unsupported (built for %d/%d/%d/%d)",
                c->kv_lora, c->qk_nope, c->qk_rope, c->v_head, MLA_KVL, MLA_NOPE, MLA_R, MLA_VH);
  if (c->HD != MLA_QD) return fail(ETXMK_EINVAL, "head_dim %d must be qk_nope + qk_rope = %d", c->HD, MLA_QD);
  if (c->NH > MLA_MAX_NH || (c->NH > MLA_G && c->NH % MLA_G)) return fail(ETXMK_EINVAL, "%d heads unsupported", c->NH);
  if (!c->moe || c->E <= 0 || c->E > MAX_E || c->E % 4 || c->TOPK <= 0 || c->TOPK > MAX_TOPK || c->TOPK > c->E)
    return fail(ETXMK_EINVAL, "experts %d / top-k %d unsupported", c->E, c->TOPK);
  if (c->n_shared < 1 || c->first_dense < 0 || c->first_dense > c->L || (c->first_dense > 0 && c->dense_I <= 0))
    return fail(ETXMK_EINVAL, "shared experts %d / dense layers %d of width %d unsupported", c->n_shared, c->first_dense, c->dense_I);
  if (c->block_size != 16 && c->block_size != 32 && c->block_size != 64)
    return fail(ETXMK_EINVAL, "block size %d unsupported (16, 32 or 64)", c->block_size);
  if (c->max_ctx <= 0 || c->max_ctx > MAX_CTX) return fail(ETXMK_EINVAL, "max_ctx %d outside 1..%d", c->max_ctx, MAX_CTX);
  if (c->batch < 1 || c->batch > MAX_B_DS) return fail(ETXMK_EINVAL, "batch %d outside 1..%d", c->batch, MAX_B_DS);
  if (c->wdtype != ETXMK_W_BF16) return fail(ETXMK_EINVAL, "DeepSeek-V2 runs bf16 weights only");
  if (c->rope_factor <= 0.0f || c->rope_orig_max <= 0 || c->beta_fast <= 0.0f || c->beta_slow <= 0.0f)
    return fail(ETXMK_EINVAL, "yarn RoPE parameters must be positive");
  if (!ds_kernel(*c))
    return fail(ETXMK_EINVAL, "no DeepSeek-V2 kernel for H %d, NH %d, MI %d, shared %d, E %d, dense I %d", c->H, c->NH,
                c->MI, ds_si(*c), c->E, c->dense_I);
  return ETXMK_OK;
}

// the symbol of the persistent kernel a step of this configuration launches, its batch capacity, or nullptr
const char* kernel_symbol(const etxmk_config& c, int* cap) {
  const int km = c.moe ? c.MI : c.I;
  if (c.arch == ETXMK_ARCH_DSV2) {
#define MK_NAME_DS(name, h_, ka_, km_, ksh_, e_, ip_, b_)                                                          \
    if (c.H == h_ && c.NH * c.v_head == ka_ && c.MI == km_ && ds_si(c) == ksh_ && c.E == e_ &&                   \
        (c.first_dense == 0 || ds_ip(c) == ip_) && c.batch <= b_) {                                               \
      *cap = b_;                                                                                                  \
      return #name;                                                                                               \
    }
    MK_DS_SHAPES(MK_NAME_DS)
#undef MK_NAME_DS
    return nullptr;
  }
  if (c.batch == 1) {
#define MK_NAME(name, h_, ka_, km_, moe_, e_, fp8_)                                                               \
    if (c.H == h_ && c.NH * c.HD == ka_ && km == km_ && (c.moe != 0) == moe_ && (!moe_ || c.E == e_) &&          \
        (c.wdtype == ETXMK_W_FP8) == fp8_) {                                                                      \
      *cap = 1;                                                                                                   \
      return #name;                                                                                               \
    }
    MK_FUSED_SHAPES_BF16(MK_NAME)
    MK_FUSED_SHAPES_FP8(MK_NAME)
#undef MK_NAME
    return nullptr;
  }
  const char* best = nullptr;
  int bc = 0;
#define MK_NAME_B(name, h_, ka_, km_, moe_, e_, fp8_, b_)                                                         \
  if (c.H == h_ && c.NH * c.HD == ka_ && km == km_ && (c.moe != 0) == moe_ && (!moe_ || c.E == e_) &&            \
      (c.wdtype == ETXMK_W_FP8) == fp8_ && c.batch <= b_ && (!best || b_ < bc)) {                                 \
    best = #name;                                                                                                 \
    bc = b_;                                                                                                      \
  }
  MK_BATCH_SHAPES_BF16(MK_NAME_B)
  MK_BATCH_SHAPES_FP8(MK_NAME_B)
#undef MK_NAME_B
  *cap = bc;
  return best;
}

// The matrix-core rule: MoE Qwen3 handles of batch capacity >= 8 whose shapes take whole tiles run their batched
// QKV, O projection, router, expert gate/up, expert down and lm_head on the matrix cores (the down outputs combined
// in a phase of their own).  The CPU oracle applies the same rule to the models of such handles.
bool mfma_rule(const etxmk_config& c) {
  const int tb = c.wdtype == ETXMK_W_FP8 ? 1024 : 512, ka = c.NH * c.HD;
  return c.arch == ETXMK_ARCH_QWEN3 && c.batch >= 8 && c.moe && c.H % tb == 0 && c.H / tb <= NWAVE && ka % tb == 0 &&
         ka / tb <= NWAVE && c.H / 512 <= NWAVE && c.E % 16 == 0 && c.MI % 256 == 0 && c.MI <= 4096 && c.V % 16 == 0;
}

// grid barriers of a launch over layers [l0, l1) (plus the head), one per phase; `batched`: the batched kernel
// (Qwen3: the attention merge is a phase of its own; with the matrix-core rule, the expert combine too)
int barriers_of(const etxmk_config& c, int l0, int l1, int head, bool batched) {
  if (c.arch == ETXMK_ARCH_DSV2) {                         // 5 attention phases, then 2 dense or 3 MoE phases
    int n = 0;
    for (int l = l0; l < l1; ++l) n += l < c.first_dense ? 7 : 8;
    return n + (head ? 1 : 0);
  }
  return ((c.moe ? 6 : 5) + (batched ? 1 : 0) + (batched && mfma_rule(c) ? 1 : 0)) * (l1 - l0) + (head ? 1 : 0);
}

int check_config(const etxmk_config* c) {
  if (!c) return fail(ETXMK_EINVAL, "config is NULL");
  if (c->H <= 0 || c->NH <= 0 || c->NKV <= 0 || c->L <= 0 || c->V <= 0) return fail(ETXMK_EINVAL, "non-positive dimension");
  if (c->arch != ETXMK_ARCH_QWEN3 && c->arch != ETXMK_ARCH_DSV2) return fail(ETXMK_EINVAL, "architecture %d unknown", c->arch);
  if (c->prefill < 0 || c->prefill > MAX_B) return fail(ETXMK_EINVAL, "prefill rows %d outside 0..%d", c->prefill, MAX_B);
  if (c->arch == ETXMK_ARCH_DSV2) {
    if (c->prefill > MAX_B_DS) return fail(ETXMK_EINVAL, "prefill rows %d outside 0..%d", c->prefill, MAX_B_DS);
    return check_ds(c);
  }
  if (c->HD != HDIM) return fail(ETXMK_EINVAL, "head_dim %d unsupported (the attention phase is built for %d)", c->HD, HDIM);
  if (c->NH % c->NKV) return fail(ETXMK_EINVAL, "NH %d not a multiple of NKV %d", c->NH, c->NKV);
  if (c->NH / c->NKV > NWAVE) return fail(ETXMK_EINVAL, "%d q heads per kv head (at most %d)", c->NH / c->NKV, NWAVE);
  if (c->H > MAX_H || !k_in(c->H, {MK_K_HIDDEN})) return fail(ETXMK_EINVAL, "hidden size %d unsupported", c->H);
  if (!k_in(c->NH * c->HD, {MK_K_ATTN})) return fail(ETXMK_EINVAL, "NH*HD %d unsupported", c->NH * c->HD);
  if (c->batch < 1 || c->batch > MAX_B) return fail(ETXMK_EINVAL, "batch %d outside 1..%d", c->batch, MAX_B);
  if (c->block_size != 16)                 // the attention tiles copy whole 16-position blocks (etx/importer/spec.py:274-281)
    return fail(ETXMK_EINVAL, "block size %d unsupported (the paged KV cache is built for 16-position blocks)", c->block_size);
  if (c->max_ctx <= 0 || c->max_ctx > MAX_CTX) return fail(ETXMK_EINVAL, "max_ctx %d outside 1..%d", c->max_ctx, MAX_CTX);
  if (c->moe) {
    if (c->E <= 0 || c->E > MAX_E || c->E % 4 || c->TOPK <= 0 || c->TOPK > MAX_TOPK || c->TOPK > c->E)
      return fail(ETXMK_EINVAL, "experts %d / top-k %d unsupported", c->E, c->TOPK);
    if (!k_in(c->MI, {MK_K_MOE}) || c->TOPK * c->MI > MAX_K) return fail(ETXMK_EINVAL, "moe intermediate %d unsupported", c->MI);
  } else {
    if (!k_in(c->I, {MK_K_INTER}) || c->I > MAX_K) return fail(ETXMK_EINVAL, "intermediate %d unsupported", c->I);
  }
  if (c->wdtype != ETXMK_W_BF16 && c->wdtype != ETXMK_W_FP8) return fail(ETXMK_EINVAL, "weight type %d unknown", c->wdtype);
  if (c->wdtype == ETXMK_W_FP8 && c->batch == 1 && !fused_kernel(*c))
    return fail(ETXMK_EINVAL, "no fp8 persistent kernel for H %d, NH*HD %d, %s %d (fp8 runs fused only)", c->H,
                c->NH * c->HD, c->moe ? "MI" : "I", c->moe ? c->MI : c->I);
  if (c->batch > 1 && !batch_kernel(*c))
    return fail(ETXMK_EINVAL, "no batched persistent kernel for batch %d, H %d, NH*HD %d, %s %d", c->batch, c->H,
                c->NH * c->HD, c->moe ? "MI" : "I", c->moe ? c->MI : c->I);
  if (c->prefill > 0 && !batch_kernel(*c, c->prefill))
    return fail(ETXMK_EINVAL, "no batched persistent kernel for %d prefill rows, H %d, NH*HD %d, %s %d", c->prefill,
                c->H, c->NH * c->HD, c->moe ? "MI" : "I", c->moe ? c->MI : c->I);
  return ETXMK_OK;
}

// Weight arena: every tensor 256-byte aligned, experts of one layer contiguous.
std::vector<TensorSlot> weight_layout(const etxmk_config* c, uint64_t* total) {
  std::vector<TensorSlot> v;
  uint64_t off = 0;
  auto add = [&](int kind, int layer, int count, int rows, int cols, int perm, int lcols = 0, int split = 0) {
    TensorSlot t{kind, layer, count, rows, cols, perm, c->wdtype == ETXMK_W_FP8 && fp8_kind(kind) ? 1 : 0, off};
    t.lcols = lcols;
    t.split = split;
    v.push_back(t);
    off = align_up(off + (uint64_t)count * t.tensor_bytes());
  };
  if (c->arch == ETXMK_ARCH_DSV2) {
    // DeepSeek-V2: kv_a_layernorm in the KNORM slot; WQKV = [q_proj; kv_a_proj_with_mqa]; WKVB = kv_b_proj; the
    // dense layers' down rows padded to whole 512 blocks
    add(ETXMK_T_EMBED, -1, 1, c->V, c->H, 0);
    add(ETXMK_T_LMHEAD, -1, 1, c->V, c->H, 1);
    add(ETXMK_T_FINAL_NORM, -1, 1, 1, c->H, 0);
    const int SI = ds_si(*c), IP = ds_ip(*c);
    for (int l = 0; l < c->L; ++l) {
      add(ETXMK_T_LN1, l, 1, 1, c->H, 0);
      add(ETXMK_T_LN2, l, 1, 1, c->H, 0);
      add(ETXMK_T_KNORM, l, 1, 1, c->kv_lora, 0);
      add(ETXMK_T_WQKV, l, 1, ds_nqa(*c), c->H, 1);
      add(ETXMK_T_WKVB, l, 1, c->NH * (c->qk_nope + c->v_head), c->kv_lora, 1, 0, 1);
      add(ETXMK_T_WO, l, 1, c->H, c->NH * c->v_head, 1);
      if (l < c->first_dense) {
        add(ETXMK_T_WGU, l, 1, 2 * c->dense_I, c->H, 1);
        add(ETXMK_T_WD, l, 1, c->H, IP, 1, c->dense_I);
      } else {
        add(ETXMK_T_ROUTER, l, 1, c->E, c->H, 1);
        add(ETXMK_T_W13, l, c->E, 2 * c->MI, c->H, 1);
        add(ETXMK_T_W2, l, c->E, c->H, c->MI, 1);
        add(ETXMK_T_WSGU, l, 1, 2 * SI, c->H, 1);
        add(ETXMK_T_WSD, l, 1, c->H, SI, 1);
      }
    }
    *total = off;
    return v;
  }
  const int NQKV = (c->NH + 2 * c->NKV) * c->HD;
  add(ETXMK_T_EMBED, -1, 1, c->V, c->H, 0);
  add(ETXMK_T_LMHEAD, -1, 1, c->V, c->H, 1);
  add(ETXMK_T_FINAL_NORM, -1, 1, 1, c->H, 0);
  for (int l = 0; l < c->L; ++l) {
    add(ETXMK_T_LN1, l, 1, 1, c->H, 0);
    add(ETXMK_T_LN2, l, 1, 1, c->H, 0);
    add(ETXMK_T_QNORM, l, 1, 1, c->HD, 0);
    add(ETXMK_T_KNORM, l, 1, 1, c->HD, 0);
    add(ETXMK_T_WQKV, l, 1, NQKV, c->H, 1);
    add(ETXMK_T_WO, l, 1, c->H, c->NH * c->HD, 1);
    if (c->moe) {
      add(ETXMK_T_ROUTER, l, 1, c->E, c->H, 1);
      add(ETXMK_T_W13, l, c->E, 2 * c->MI, c->H, 1);
      add(ETXMK_T_W2, l, c->E, c->H, c->MI, 1);
    } else {
      add(ETXMK_T_WGU, l, 1, 2 * c->I, c->H, 1);
      add(ETXMK_T_WD, l, 1, c->H, c->I, 1);
    }
  }
  *total = off;
  return v;
}

// paged KV: every sequence of the batch owns up to nbps blocks of one shared pool
int nbps_of(const etxmk_config* c) { return (c->max_ctx + c->block_size - 1) / c->block_size; }
int nblocks_of(const etxmk_config* c) { return c->batch * nbps_of(c); }
int rows_of(const etxmk_config& c) { return c.batch > c.prefill ? c.batch : c.prefill; }

// per layer: K and V pools of this many elements each (DeepSeek-V2: one latent pool)
uint64_t kv_layer_elems(const etxmk_config* c) {
  if (c->arch == ETXMK_ARCH_DSV2) return (uint64_t)nblocks_of(c) * c->block_size * MLA_CD;
  return (uint64_t)nblocks_of(c) * c->block_size * c->NKV * c->HD;
}
int kv_pools(const etxmk_config* c) { return c->arch == ETXMK_ARCH_DSV2 ? 1 : 2; }

struct WsLayout {
  uint64_t x, x16, qkv, o, o16, logits, hbuf, h16, ys, apart, acnt, amax, bar, abort_w, tokens, out_tokens, btab, rcos, rsin,
      layers, h16d, qc, h16s, sink, total;
};

WsLayout ws_layout(const etxmk_config* c) {
  WsLayout w{};
  uint64_t off = 0;
  auto take = [&](uint64_t bytes) { const uint64_t o = off; off = align_up(off + bytes); return o; };
  const bool ds = c->arch == ETXMK_ARCH_DSV2;
  const int NQKV = nqkv_of(*c), KA = ds ? c->NH * c->v_head : c->NH * c->HD;
  const uint64_t B = (uint64_t)rows_of(*c);   // activation rows: sequences, or prefill positions
  w.x = take(4ull * c->H * B);
  w.x16 = take(2ull * c->H * B);
  w.qkv = take(4ull * NQKV * B);
  w.o = take(4ull * KA * B);
  w.o16 = take(2ull * KA * B);
  w.logits = take(4ull * (c->E > 0 ? c->E : 1) * B);
  const int hb = c->moe ? c->TOPK * c->MI : c->I;
  w.hbuf = take(4ull * (hb > 0 ? hb : 1) * B);
  w.h16 = take(2ull * (hb > 0 ? hb : 1) * B);
  w.ys = take(2ull * (c->moe ? c->TOPK : 1) * c->H * B);   // matrix-core expert down: weighted outputs per pair
  w.apart = take(4ull * c->NH * MAX_CHUNKS * (ds ? MLA_PART : PART) * B);
  w.acnt = take(4ull * 64 * 2 * (ds ? ds_nhg(*c) : c->NKV) * B); // one 256-byte line per (sequence, kv head / head group, half)
  w.amax = take(256ull * B);             // one 256-byte line per sequence
  w.bar = take(4 * 64 * 17);          // 8 group counters, 1 global counter, 8 release flags; 256 B apart
  w.abort_w = take(4);
  w.tokens = take(4ull * (c->max_ctx + 1) * c->batch);
  w.out_tokens = take(4ull * (c->max_ctx + 1) * c->batch);
  w.btab = take(4ull * nblocks_of(c));
  const int rhalf = ds ? c->qk_rope / 2 : c->HD / 2;
  w.rcos = take(4ull * c->max_ctx * rhalf);
  w.rsin = take(4ull * c->max_ctx * rhalf);
  w.layers = take(sizeof(LayerW) * (uint64_t)c->L);
  if (ds) {
    w.h16d = take(2ull * (c->first_dense > 0 ? ds_ip(*c) : 8) * B);
    w.qc = take(4ull * c->L * c->NH * c->kv_lora * B);   // one buffer per layer (read through the scalar cache)
    w.h16s = take(2ull * ds_si(*c) * B);
  } else {
    w.h16d = w.h16;
  }
  w.sink = take(4ull * SINK_WAVES * 64);
  w.total = off;
  return w;
}

uint64_t acnt_bytes(const etxmk_config& c) { return 4ull * 64 * 2 * (is_ds(c) ? ds_nhg(c) : c.NKV) * rows_of(c); }

// DeepseekV2YarnRotaryEmbedding tables (reference_decode.py:85-118) in the steps the reference's numpy takes in
// float32: the correction range in double, the ramp, mask and inverse frequencies in float, then cos and sin of
// t * inv times the ratio of the two yarn mscales (first half only: emb = cat(freqs, freqs)); kept in fp32
void yarn_tables(const etxmk_config& c, float* cs, float* sn) {
  const int dim = c.qk_rope, half = dim / 2;
  const double base = c.theta, two_pi = 2.0 * 3.141592653589793;
  auto mscale = [](double scale, double m) { return scale <= 1.0 ? 1.0 : 0.1 * m * log(scale) + 1.0; };
  const double lowd = (dim * log(c.rope_orig_max / (c.beta_fast * two_pi))) / (2.0 * log(base));
  const double highd = (dim * log(c.rope_orig_max / (c.beta_slow * two_pi))) / (2.0 * log(base));
  int low = (int)floor(lowd), high = (int)ceil(highd);
  if (low < 0) low = 0;
  if (high > dim - 1) high = dim - 1;
  const float span = low == high ? (float)((double)high + 0.001 - (double)low) : (float)(high - low);
  const float ms = (float)(mscale(c.rope_factor, c.rope_mscale) / mscale(c.rope_factor, c.rope_mscale_all));
  std::vector<float> inv(half);
  for (int i = 0; i < half; ++i) {
    const float e = (float)(2 * i) / (float)dim;
    const float pw = powf((float)base, e);
    const float extra = 1.0f / pw, inter = 1.0f / ((float)c.rope_factor * pw);
    float ramp = ((float)i - (float)low) / span;
    ramp = ramp < 0.0f ? 0.0f : ramp > 1.0f ? 1.0f : ramp;
    const float mask = 1.0f - ramp;
    inv[i] = inter * (1.0f - mask) + extra * mask;
  }
  for (int t = 0; t < c.max_ctx; ++t)
    for (int i = 0; i < half; ++i) {
      const float f = (float)t * inv[i];
      cs[(size_t)t * half + i] = cosf(f) * ms;
      sn[(size_t)t * half + i] = sinf(f) * ms;
    }
}

// ---------------------------------------------------------------- allocation-free step (etxmk_step_static)
// The scratch of a single-sequence step (activations, attention chunk partials, attention arrival counters, the argmax
// key, the grid-barrier words) in one file-scope device array instead of the caller's workspace.  Each GPU the library
// runs on holds its own copy until the process ends; its device address comes from hipGetSymbolAddress, taken once per
// device with that device current (host code never uses the array's name as an address).
constexpr uint64_t STATIC_SCRATCH_BYTES = 4ull << 20;
constexpr int MAX_DEVICES = 64;

struct StaticLayout {
  uint64_t bar, acnt, amax, zero_end;     // counters first: [0, zero_end) is cleared by every call
  uint64_t x, qkv, o, logits, hbuf, apart, total;
};

StaticLayout static_layout(const etxmk_config& c) {
  StaticLayout w{};
  uint64_t off = 0;
  auto take = [&](uint64_t bytes) { const uint64_t o = off; off = align_up(off + bytes); return o; };
  w.bar = take(4 * 64 * 17);
  w.acnt = take(4ull * 64 * 2 * c.NKV);
  w.amax = take(256);
  w.zero_end = off;
  const int hb = c.moe ? c.TOPK * c.MI : c.I;
  w.x = take(4ull * c.H);
  w.qkv = take(4ull * nqkv_of(c));
  w.o = take(4ull * c.NH * c.HD);
  w.logits = take(4ull * (c.E > 0 ? c.E : 1));
  w.hbuf = take(4ull * (hb > 0 ? hb : 1));
  w.apart = take(4ull * c.NH * MAX_CHUNKS * PART);
  w.total = off;
  return w;
}

// pointers of the step's scratch buffers when they do not come from the workspace
struct ScratchView {
  uint8_t* base;
  StaticLayout lay;
};

}  // namespace

struct etxmk_handle {
  etxmk_config c;
  std::vector<TensorSlot> slots;
  uint64_t wbytes = 0;
  WsLayout ws{};
  uint8_t* w = nullptr;
  uint8_t* kv = nullptr;
  uint8_t* wsp = nullptr;
  int fused = 1;
  int nwg = 0;
  int ncu = 0;
  uint32_t bar_epoch = 0;
  float* dump_x = nullptr;
  int32_t* dump_ids = nullptr;
  float* dump_wts = nullptr;
  float* dump_logits = nullptr;
  uint64_t* trace = nullptr;
  std::vector<int32_t> btab_host;
  int32_t* stop_host = nullptr;          // pinned, device-mapped host word: nonzero asks a running step to stop
  int32_t* stop_dev = nullptr;           // its device address
  uint64_t spin_ticks = SPIN_TICKS_DEFAULT;
  uint32_t poll_mask = 255;

  const TensorSlot* slot(int kind, int layer) const {
    for (const auto& s : slots)
      if (s.kind == kind && s.layer == layer) return &s;
    return nullptr;
  }
  template <class T> T* wsptr(uint64_t off) const { return (T*)(wsp + off); }
  const uint8_t* wt(int kind, int layer) const {
    const TensorSlot* s = slot(kind, layer);
    return s ? (const uint8_t*)(w + s->off) : nullptr;
  }
  int barriers(int l0, int l1, int head, bool batched) const { return barriers_of(c, l0, l1, head, batched); }
};

static __device__ __align__(256) uint8_t scratch[STATIC_SCRATCH_BYTES];

namespace {
std::mutex g_scratch_mu;
uint8_t* g_scratch_ptr[MAX_DEVICES];

// the calling thread's current device's copy of `scratch` (resolved on the first call on that device)
int scratch_ptr(uint8_t** out) {
  int dev = 0;
  HIPCHK(hipGetDevice(&dev));
  if (dev < 0 || dev >= MAX_DEVICES) return fail(ETXMK_EINVAL, "device %d outside 0..%d", dev, MAX_DEVICES - 1);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    HIPCHK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    g_scratch_ptr[dev] = (uint8_t*)ptr;
  }
  *out = g_scratch_ptr[dev];
  return ETXMK_OK;
}
}  // namespace

extern "C" {

int etxmk_abi_version(void) { return ETXMK_ABI_VERSION; }
const char* etxmk_last_error(void) { return g_err; }

int etxmk_weight_bytes(const etxmk_config* cfg, uint64_t* bytes) {
  if (int r = check_config(cfg)) return r;
  if (!bytes) return fail(ETXMK_EINVAL, "bytes is NULL");
  weight_layout(cfg, bytes);
  return ETXMK_OK;
}

int etxmk_kv_bytes(const etxmk_config* cfg, uint64_t* bytes) {
  if (int r = check_config(cfg)) return r;
  if (!bytes) return fail(ETXMK_EINVAL, "bytes is NULL");
  *bytes = 2ull * kv_pools(cfg) * kv_layer_elems(cfg) * (uint64_t)cfg->L;
  return ETXMK_OK;
}

int etxmk_workspace_bytes(const etxmk_config* cfg, uint64_t* bytes) {
  if (int r = check_config(cfg)) return r;
  if (!bytes) return fail(ETXMK_EINVAL, "bytes is NULL");
  *bytes = ws_layout(cfg).total;
  return ETXMK_OK;
}

int etxmk_plan(const etxmk_config* cfg, int32_t fused, etxmk_plan_info* out) {
  if (int r = check_config(cfg)) return r;
  if (!out) return fail(ETXMK_EINVAL, "out is NULL");
  const etxmk_config& c = *cfg;
  if (!fused && (c.batch > 1 || c.wdtype == ETXMK_W_FP8 || c.arch == ETXMK_ARCH_DSV2))
    return fail(ETXMK_EINVAL, "the unfused mode runs bf16 Qwen3 handles at batch 1 only");
  memset(out, 0, sizeof *out);
  int cap = 1;
  const char* sym = fused ? kernel_symbol(c, &cap) : "unfused";
  if (!sym) return fail(ETXMK_EINVAL, "no persistent kernel for this shape (use the unfused mode)");
  snprintf(out->kernel, sizeof out->kernel, "%s", sym);
  out->barriers_per_step = barriers_of(c, 0, c.L, 1, c.batch > 1);
  out->threads = NT;
  out->batch_capacity = cap;
  out->matrix_cores = fused && mfma_rule(c) ? 1 : 0;
  weight_layout(cfg, &out->weight_bytes);
  out->kv_bytes = 2ull * kv_pools(cfg) * kv_layer_elems(cfg) * (uint64_t)c.L;
  out->workspace_bytes = ws_layout(cfg).total;
  return ETXMK_OK;
}

int etxmk_create(const etxmk_config* cfg, etxmk_handle** out) {
  if (int r = check_config(cfg)) return r;
  if (!out) return fail(ETXMK_EINVAL, "out is NULL");
  etxmk_handle* h = new etxmk_handle();
  h->c = *cfg;
  h->slots = weight_layout(cfg, &h->wbytes);
  h->ws = ws_layout(cfg);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&h->ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
    delete h;
    return fail(ETXMK_EHIP, "no HIP device");
  }
  h->nwg = h->ncu;
  // the host's stop word lives in pinned host memory mapped into the device's address space, so the host can set it
  // with a plain store while a persistent launch holds every CU (a copy or fill would need a queue slot behind it)
  if (hipHostMalloc((void**)&h->stop_host, 4, hipHostMallocMapped) != hipSuccess ||
      hipHostGetDevicePointer((void**)&h->stop_dev, h->stop_host, 0) != hipSuccess) {
    if (h->stop_host) (void)hipHostFree(h->stop_host);
    delete h;
    return fail(ETXMK_EHIP, "pinned stop word: %s", hipGetErrorString(hipGetLastError()));
  }
  __atomic_store_n(h->stop_host, 0, __ATOMIC_SEQ_CST);
  *out = h;
  return ETXMK_OK;
}

int etxmk_destroy(etxmk_handle* h) {
  if (!h) return ETXMK_OK;
  if (h->stop_host) (void)hipHostFree(h->stop_host);
  delete h;
  return ETXMK_OK;
}

int etxmk_bind(etxmk_handle* h, void* weights, void* kv, void* workspace) {
  if (!h || !weights || !kv || !workspace) return fail(ETXMK_EINVAL, "NULL handle or buffer");
  if (((uintptr_t)weights | (uintptr_t)kv | (uintptr_t)workspace) & (ALIGN - 1))
    return fail(ETXMK_EINVAL, "buffers must be %llu-byte aligned", (unsigned long long)ALIGN);
  h->w = (uint8_t*)weights;
  h->kv = (uint8_t*)kv;
  h->wsp = (uint8_t*)workspace;
  const etxmk_config& c = h->c;
  // per-layer pointer table
  std::vector<LayerW> lw(c.L);
  const uint64_t kvl = kv_layer_elems(&c);
  const bool ds = is_ds(c);
  for (int l = 0; l < c.L; ++l) {
    LayerW& y = lw[l];
    y.ln1 = (const uint16_t*)h->wt(ETXMK_T_LN1, l);
    y.ln2 = (const uint16_t*)h->wt(ETXMK_T_LN2, l);
    y.qn = (const uint16_t*)h->wt(ETXMK_T_QNORM, l);
    y.kn = (const uint16_t*)h->wt(ETXMK_T_KNORM, l);
    y.wqkv = h->wt(ETXMK_T_WQKV, l);
    y.wo = h->wt(ETXMK_T_WO, l);
    y.wr = h->wt(ETXMK_T_ROUTER, l);
    y.w13 = h->wt(ETXMK_T_W13, l);
    y.w2 = h->wt(ETXMK_T_W2, l);
    y.wgu = h->wt(ETXMK_T_WGU, l);
    y.wd = h->wt(ETXMK_T_WD, l);
    y.kc = (uint16_t*)h->kv + (uint64_t)l * kv_pools(&c) * kvl;
    y.vc = ds ? nullptr : y.kc + kvl;
    if (ds) {
      const TensorSlot* kvb = h->slot(ETXMK_T_WKVB, l);
      y.wuk = h->w + kvb->off;
      y.wuv = y.wuk + 2ull * c.NH * c.kv_lora * c.qk_nope;
      y.wsgu = h->wt(ETXMK_T_WSGU, l);
      y.wsd = h->wt(ETXMK_T_WSD, l);
    }
  }
  HIPCHK(hipMemcpy(h->wsp + h->ws.layers, lw.data(), sizeof(LayerW) * c.L, hipMemcpyHostToDevice));
  const int half = ds ? c.qk_rope / 2 : c.HD / 2;
  std::vector<float> cs((size_t)c.max_ctx * half), sn((size_t)c.max_ctx * half);
  if (ds) {
    yarn_tables(c, cs.data(), sn.data());
  } else {
    // RoPE tables, bf16 values in fp32 (ref_numpy.py:76-81; host.hip:164-178)
    for (int i = 0; i < half; ++i) {
      const float inv = 1.0f / powf(c.theta, (float)(2 * i) / (float)c.HD);
      for (int t = 0; t < c.max_ctx; ++t) {
        const float f = (float)t * inv;
        auto rb = [](float x) { uint32_t u; memcpy(&u, &x, 4); u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u; float r; memcpy(&r, &u, 4); return r; };
        cs[(size_t)t * half + i] = rb(cosf(f));
        sn[(size_t)t * half + i] = rb(sinf(f));
      }
    }
  }
  HIPCHK(hipMemcpy(h->wsp + h->ws.rcos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
  HIPCHK(hipMemcpy(h->wsp + h->ws.rsin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
  // identity block tables (sequence b owns blocks [b*nbps, (b+1)*nbps)), counters and token buffers cleared
  h->btab_host.resize(nblocks_of(&c));
  for (int i = 0; i < (int)h->btab_host.size(); ++i) h->btab_host[i] = i;
  HIPCHK(hipMemcpy(h->wsp + h->ws.btab, h->btab_host.data(), h->btab_host.size() * 4, hipMemcpyHostToDevice));
  HIPCHK(hipMemset(h->wsp + h->ws.bar, 0, 4 * 64 * 17));
  HIPCHK(hipMemset(h->wsp + h->ws.abort_w, 0, 4));
  HIPCHK(hipMemset(h->wsp + h->ws.tokens, 0, 4ull * (c.max_ctx + 1) * c.batch));
  HIPCHK(hipMemset(h->wsp + h->ws.out_tokens, 0, 4ull * (c.max_ctx + 1) * c.batch));
  HIPCHK(hipMemset(h->wsp + h->ws.x, 0, 4ull * c.H * rows_of(c)));
  HIPCHK(hipMemset(h->wsp + h->ws.x16, 0, 2ull * c.H * rows_of(c)));
  HIPCHK(hipMemset(h->wsp + h->ws.acnt, 0, acnt_bytes(c)));
  if (ds) HIPCHK(hipMemset(h->wsp + h->ws.h16d, 0, 2ull * (c.first_dense > 0 ? ds_ip(c) : 8) * rows_of(c)));  // zero pads
  h->bar_epoch = 0;
  return ETXMK_OK;
}

int etxmk_tensor_info(etxmk_handle* h, int kind, int layer, int expert, uint64_t* offset, int32_t* rows, int32_t* cols,
                      int32_t* permuted) {
  if (!h) return fail(ETXMK_EINVAL, "NULL handle");
  const bool global = kind == ETXMK_T_EMBED || kind == ETXMK_T_LMHEAD || kind == ETXMK_T_FINAL_NORM;
  const TensorSlot* s = h->slot(kind, global ? -1 : layer);
  if (!s) return fail(ETXMK_EINVAL, "no tensor kind %d layer %d", kind, layer);
  if (expert < 0 || expert >= s->count) return fail(ETXMK_EINVAL, "expert %d outside 0..%d", expert, s->count - 1);
  if (offset) *offset = s->off + (uint64_t)expert * s->tensor_bytes();
  if (rows) *rows = s->rows;
  if (cols) *cols = s->logical_cols();
  if (permuted) *permuted = s->perm;
  return ETXMK_OK;
}

int etxmk_tensor_format(etxmk_handle* h, int kind, int layer, int32_t* wdtype, uint64_t* row_bytes) {
  if (!h) return fail(ETXMK_EINVAL, "NULL handle");
  const bool global = kind == ETXMK_T_EMBED || kind == ETXMK_T_LMHEAD || kind == ETXMK_T_FINAL_NORM;
  const TensorSlot* s = h->slot(kind, global ? -1 : layer);
  if (!s) return fail(ETXMK_EINVAL, "no tensor kind %d layer %d", kind, layer);
  if (wdtype) *wdtype = s->fp8 ? ETXMK_W_FP8 : ETXMK_W_BF16;
  if (row_bytes) *row_bytes = s->row_bytes();
  return ETXMK_OK;
}

// fp8 rows of n_t tensors (rows x cols) at dst, from the seeded generator (src null) or natural bf16 rows
static int quantize(uint8_t* dst, const uint16_t* src, uint64_t seed, uint64_t sid0, int n_t, int rows, int cols,
                    float scale, hipStream_t st) {
  const size_t nrows = (size_t)n_t * rows, blocks = (nrows + 3) / 4;   // 4 waves per block, one row each
  hipLaunchKernelGGL(etxmk_quant_rows, dim3((unsigned)(blocks < 65536 ? blocks : 65536)), dim3(256), 0, st, dst, src,
                     seed, sid0, n_t, rows, cols, scale);
  HIPCHK(hipGetLastError());
  return ETXMK_OK;
}

int etxmk_init_weights_seeded(etxmk_handle* h, uint64_t seed, float scale, void* stream) {
  if (!h || !h->w) return fail(ETXMK_EUNBOUND, "handle not bound");
  hipStream_t st = (hipStream_t)stream;
  for (const TensorSlot& s : h->slots) {
    uint16_t* dst = (uint16_t*)(h->w + s.off);
    const size_t n = (size_t)s.count * s.rows * s.cols;
    const bool norm = s.kind >= ETXMK_T_LN1;
    if (s.fp8) {
      if (int r = quantize(h->w + s.off, nullptr, seed, stream_id(s.kind, s.layer, 0), s.count, s.rows, s.cols, scale, st))
        return r;
      continue;
    }
    if (norm) {
      hipLaunchKernelGGL(etxmk_fill_u16, dim3(64), dim3(256), 0, st, dst, n, (uint16_t)0x3F80);
    } else if (s.split) {
      const etxmk_config& c = h->c;
      hipLaunchKernelGGL(etxmk_pack_kvb, dim3((unsigned)((n + 255) / 256 < 65536 ? (n + 255) / 256 : 65536)), dim3(256), 0,
                         st, dst, (const uint16_t*)nullptr, seed, stream_id(s.kind, s.layer, 0), c.NH, c.qk_nope,
                         c.v_head, c.kv_lora, scale);
    } else {
      if (n % 8) return fail(ETXMK_EINVAL, "tensor kind %d has %zu elements (not a multiple of 8)", s.kind, n);
      const size_t blocks = (n / 8 + 255) / 256;
      hipLaunchKernelGGL(etxmk_gen_weights, dim3((unsigned)(blocks < 65536 ? blocks : 65536)), dim3(256), 0, st, dst, seed,
                         stream_id(s.kind, s.layer, 0), s.count, s.rows, s.cols, s.logical_cols(), s.perm, scale);
    }
    HIPCHK(hipGetLastError());
  }
  return ETXMK_OK;
}

int etxmk_load_tensor(etxmk_handle* h, int kind, int layer, int expert, const void* src, void* stream) {
  if (!h || !h->w) return fail(ETXMK_EUNBOUND, "handle not bound");
  uint64_t off;
  int32_t rows, cols, perm;
  if (int r = etxmk_tensor_info(h, kind, layer, expert, &off, &rows, &cols, &perm)) return r;
  if (!src) return fail(ETXMK_EINVAL, "src is NULL");
  hipStream_t st = (hipStream_t)stream;
  const bool global = kind == ETXMK_T_EMBED || kind == ETXMK_T_LMHEAD || kind == ETXMK_T_FINAL_NORM;
  const TensorSlot* ts = h->slot(kind, global ? -1 : layer);
  if (ts->fp8) return quantize(h->w + off, (const uint16_t*)src, 0, 0, 1, rows, cols, 0.0f, st);
  if (ts->split) {
    const etxmk_config& c = h->c;
    const size_t n = (size_t)rows * cols;
    hipLaunchKernelGGL(etxmk_pack_kvb, dim3((unsigned)((n + 255) / 256 < 65536 ? (n + 255) / 256 : 65536)), dim3(256), 0, st,
                       (uint16_t*)(h->w + off), (const uint16_t*)src, (uint64_t)0, (uint64_t)0, c.NH, c.qk_nope, c.v_head,
                       c.kv_lora, 0.0f);
    HIPCHK(hipGetLastError());
  } else if (perm) {
    const size_t n = (size_t)rows * ts->cols;
    hipLaunchKernelGGL(etxmk_pack_rows, dim3((unsigned)((n + 255) / 256 < 65536 ? (n + 255) / 256 : 65536)), dim3(256), 0, st,
                       (uint16_t*)(h->w + off), (const uint16_t*)src, rows, ts->cols, cols);
    HIPCHK(hipGetLastError());
  } else {
    HIPCHK(hipMemcpyAsync(h->w + off, src, (size_t)rows * cols * 2, hipMemcpyDeviceToDevice, st));
  }
  return ETXMK_OK;
}

int etxmk_set_block_table(etxmk_handle* h, const int32_t* table, int32_t n, void* stream) {
  if (!h || !h->wsp) return fail(ETXMK_EUNBOUND, "handle not bound");
  const int nb = nblocks_of(&h->c);
  if (!table || n <= 0 || n > nb) return fail(ETXMK_EINVAL, "block table length %d outside 1..%d", n, nb);
  std::vector<int32_t> next(h->btab_host);
  for (int i = 0; i < n; ++i) {
    if (table[i] < 0 || table[i] >= nb) return fail(ETXMK_EINVAL, "block %d maps to %d outside 0..%d", i, table[i], nb - 1);
    next[i] = table[i];
  }
  std::vector<char> seen(nb, 0);                 // no physical block may serve two (sequence, logical block) slots
  for (int i = 0; i < nb; ++i) {
    if (seen[next[i]]) return fail(ETXMK_EINVAL, "physical block %d used twice", next[i]);
    seen[next[i]] = 1;
  }
  for (int i = 0; i < n; ++i) h->btab_host[i] = table[i];
  HIPCHK(hipMemcpyAsync(h->wsp + h->ws.btab, h->btab_host.data(), 4ull * n, hipMemcpyHostToDevice, (hipStream_t)stream));
  HIPCHK(hipStreamSynchronize((hipStream_t)stream));
  return ETXMK_OK;
}

int etxmk_fill_kv_seeded_seq(etxmk_handle* h, uint64_t seed, int32_t seq, int32_t npos, void* stream) {
  if (!h || !h->kv) return fail(ETXMK_EUNBOUND, "handle not bound");
  const etxmk_config& c = h->c;
  if (seq < 0 || seq >= c.batch) return fail(ETXMK_EINVAL, "sequence %d outside 0..%d", seq, c.batch - 1);
  if (npos < 0 || npos > c.max_ctx) return fail(ETXMK_EINVAL, "npos %d outside 0..%d", npos, c.max_ctx);
  if (npos == 0) return ETXMK_OK;
  const uint64_t kvl = kv_layer_elems(&c);
  if (is_ds(c)) {                          // the latent cache (stream kind 10, as the K cache of the Qwen3 path)
    for (int l = 0; l < c.L; ++l) {
      uint16_t* kc = (uint16_t*)h->kv + (uint64_t)l * kvl;
      const size_t n = (size_t)npos * MLA_CD;
      hipLaunchKernelGGL(etxmk_gen_latent, dim3((unsigned)((n + 255) / 256 < 65536 ? (n + 255) / 256 : 65536)), dim3(256), 0,
                         (hipStream_t)stream, kc, h->wsptr<const int32_t>(h->ws.btab) + (size_t)seq * nbps_of(&c),
                         stream_key(seed, stream_id(10, l, seq)), npos, MLA_CD, c.block_size);
      HIPCHK(hipGetLastError());
    }
    return ETXMK_OK;
  }
  for (int l = 0; l < c.L; ++l) {
    uint16_t* kc = (uint16_t*)h->kv + (uint64_t)l * 2 * kvl;
    const size_t n = (size_t)npos * c.NKV * c.HD;
    hipLaunchKernelGGL(etxmk_gen_kv, dim3((unsigned)((n + 255) / 256 < 65536 ? (n + 255) / 256 : 65536)), dim3(256), 0,
                       (hipStream_t)stream, kc, kc + kvl, h->wsptr<const int32_t>(h->ws.btab) + (size_t)seq * nbps_of(&c),
                       stream_key(seed, stream_id(10, l, seq)), stream_key(seed, stream_id(11, l, seq)), npos, c.NKV,
                       c.HD, c.block_size);
    HIPCHK(hipGetLastError());
  }
  return ETXMK_OK;
}

int etxmk_fill_kv_seeded(etxmk_handle* h, uint64_t seed, int32_t npos, void* stream) {
  return etxmk_fill_kv_seeded_seq(h, seed, 0, npos, stream);
}

int etxmk_set_tokens_seq(etxmk_handle* h, int32_t seq, const int32_t* tokens, int32_t n, void* stream) {
  if (!h || !h->wsp) return fail(ETXMK_EUNBOUND, "handle not bound");
  if (seq < 0 || seq >= h->c.batch) return fail(ETXMK_EINVAL, "sequence %d outside 0..%d", seq, h->c.batch - 1);
  if (!tokens || n < 0 || n > h->c.max_ctx + 1) return fail(ETXMK_EINVAL, "token count %d outside 0..%d", n, h->c.max_ctx + 1);
  for (int i = 0; i < n; ++i)
    if (tokens[i] < 0 || tokens[i] >= h->c.V) return fail(ETXMK_EINVAL, "token %d = %d outside 0..%d", i, tokens[i], h->c.V - 1);
  HIPCHK(hipMemcpyAsync(h->wsp + h->ws.tokens + 4ull * (h->c.max_ctx + 1) * seq, tokens, 4ull * n, hipMemcpyHostToDevice,
                        (hipStream_t)stream));
  HIPCHK(hipStreamSynchronize((hipStream_t)stream));
  return ETXMK_OK;
}

int etxmk_set_tokens(etxmk_handle* h, const int32_t* tokens, int32_t n, void* stream) {
  return etxmk_set_tokens_seq(h, 0, tokens, n, stream);
}

int etxmk_read_tokens_seq(etxmk_handle* h, int32_t seq, int32_t* out, int32_t n, void* stream) {
  if (!h || !h->wsp) return fail(ETXMK_EUNBOUND, "handle not bound");
  if (seq < 0 || seq >= h->c.batch) return fail(ETXMK_EINVAL, "sequence %d outside 0..%d", seq, h->c.batch - 1);
  if (!out || n < 0 || n > h->c.max_ctx + 1) return fail(ETXMK_EINVAL, "token count %d outside 0..%d", n, h->c.max_ctx + 1);
  HIPCHK(hipMemcpyAsync(out, h->wsp + h->ws.out_tokens + 4ull * (h->c.max_ctx + 1) * seq, 4ull * n, hipMemcpyDeviceToHost,
                        (hipStream_t)stream));
  HIPCHK(hipStreamSynchronize((hipStream_t)stream));
  return ETXMK_OK;
}

int etxmk_read_tokens(etxmk_handle* h, int32_t* out, int32_t n, void* stream) {
  return etxmk_read_tokens_seq(h, 0, out, n, stream);
}

int etxmk_set_residual(etxmk_handle* h, const float* x, void* stream) {
  if (!h || !h->wsp) return fail(ETXMK_EUNBOUND, "handle not bound");
  if (h->c.batch != 1 || is_ds(h->c)) return fail(ETXMK_EINVAL, "the residual entry points serve single-sequence Qwen3 handles");
  if (!x) return fail(ETXMK_EINVAL, "x is NULL");
  HIPCHK(hipMemcpyAsync(h->wsp + h->ws.x, x, 4ull * h->c.H, hipMemcpyHostToDevice, (hipStream_t)stream));
  HIPCHK(hipStreamSynchronize((hipStream_t)stream));
  return ETXMK_OK;
}

int etxmk_read_residual(etxmk_handle* h, float* x, void* stream) {
  if (!h || !h->wsp) return fail(ETXMK_EUNBOUND, "handle not bound");
  if (h->c.batch != 1 || is_ds(h->c)) return fail(ETXMK_EINVAL, "the residual entry points serve single-sequence Qwen3 handles");
  if (!x) return fail(ETXMK_EINVAL, "x is NULL");
  HIPCHK(hipMemcpyAsync(x, h->wsp + h->ws.x, 4ull * h->c.H, hipMemcpyDeviceToHost, (hipStream_t)stream));
  HIPCHK(hipStreamSynchronize((hipStream_t)stream));
  return ETXMK_OK;
}

int etxmk_set_fused(etxmk_handle* h, int32_t fused) {
  if (!h) return fail(ETXMK_EINVAL, "NULL handle");
  h->fused = fused ? 1 : 0;
  return ETXMK_OK;
}

int etxmk_set_grid(etxmk_handle* h, int32_t workgroups) {
  if (!h) return fail(ETXMK_EINVAL, "NULL handle");
  const etxmk_config& c = h->c;
  const int need = 8;                       // the grid barrier spreads arrivals over 8 groups
  const int wg = workgroups > 0 ? workgroups : h->ncu;
  if (wg < need || wg > h->ncu) return fail(ETXMK_EINVAL, "workgroups %d outside %d..%d", wg, need, h->ncu);
  if (wg != h->nwg && h->wsp) {            // barrier counters assume a fixed grid: restart them
    HIPCHK(hipDeviceSynchronize());
    HIPCHK(hipMemset(h->wsp + h->ws.bar, 0, 4 * 64 * 17));
    h->bar_epoch = 0;
  }
  h->nwg = wg;
  return ETXMK_OK;
}

int etxmk_set_dump(etxmk_handle* h, float* x_layers, int32_t* topk_ids, float* topk_w, float* router_logits) {
  if (!h) return fail(ETXMK_EINVAL, "NULL handle");
  h->dump_x = x_layers;
  h->dump_ids = topk_ids;
  h->dump_wts = topk_w;
  h->dump_logits = router_logits;
  return ETXMK_OK;
}

int etxmk_set_trace(etxmk_handle* h, uint64_t* stamps) {
  if (!h) return fail(ETXMK_EINVAL, "NULL handle");
  h->trace = stamps;
  return ETXMK_OK;
}

int etxmk_barriers_per_step(etxmk_handle* h, int32_t* n) {
  if (!h || !n) return fail(ETXMK_EINVAL, "NULL argument");
  *n = h->barriers(0, h->c.L, 1, h->c.batch > 1);
  return ETXMK_OK;
}

// pseq >= 0: prefill of sequence pseq, rows b = positions posv[0] + b (nrows of them)
// sv: the step's scratch buffers come from sv (etxmk_step_static) instead of the workspace
static int launch(etxmk_handle* h, const int32_t* posv, int pos, int write_next, int l0, int l1, int embed, int head,
                  hipStream_t st, int pseq = -1, int nrows = 0, const ScratchView* sv = nullptr) {
  if (!h || !h->wsp) return fail(ETXMK_EUNBOUND, "handle not bound");
  const etxmk_config& c = h->c;
  const bool ds = is_ds(c), pf = pseq >= 0;
  // DeepSeek-V2 runs its batched kernel, a single sequence as a batch of one; prefill runs the batched kernel
  const bool batched = c.batch > 1 || ds || pf;
  if (!pf) nrows = batched ? c.batch : 1;
  if (c.batch > 1 && !posv) return fail(ETXMK_EINVAL, "a batched handle steps through etxmk_step_batch");
  if (c.batch == 1 && posv && !pf) pos = posv[0];
  int32_t pos1 = pos;
  if (batched && !posv) posv = &pos1;
  for (int b = 0; b < nrows; ++b) {
    const int q = batched ? posv[b] : pos;
    if (q < 0 || q >= c.max_ctx) return fail(ETXMK_EINVAL, "sequence %d position %d outside 0..%d", pf ? pseq : b, q,
                                             c.max_ctx - 1);
  }
  if (l0 < 0 || l1 > c.L || l0 >= l1) return fail(ETXMK_EINVAL, "layer range [%d, %d) outside [0, %d)", l0, l1, c.L);
  const int need = 8;                       // the grid barrier spreads arrivals over 8 groups
  if (h->nwg < need) return fail(ETXMK_EINVAL, "grid of %d workgroups is below the %d the grid barrier needs", h->nwg, need);
  if (!h->fused && c.wdtype == ETXMK_W_FP8) return fail(ETXMK_EINVAL, "fp8 weights run the persistent kernel only");
  if (batched) {
    if (!h->fused) return fail(ETXMK_EINVAL, "batched handles run the persistent kernel only");
    if (!embed || !head) return fail(ETXMK_EINVAL, "batched handles run whole steps");
    if ((int64_t)h->nwg * NWAVE * (RES_ROWS / NWAVE) < c.H)
      return fail(ETXMK_EINVAL, "grid of %d workgroups too small for H %d at batch > 1 (at least %d)", h->nwg, c.H,
                  (c.H + RES_ROWS - 1) / RES_ROWS);
  }
  Params p{};
  p.H = c.H; p.NH = c.NH; p.NKV = c.NKV; p.HD = c.HD; p.I = c.I; p.E = c.E; p.TOPK = c.TOPK; p.MI = c.MI; p.L = c.L; p.V = c.V;
  p.moe = c.moe; p.qk_norm = c.qk_norm; p.norm_topk = c.norm_topk; p.BS = c.block_size; p.max_ctx = c.max_ctx;
  p.nblocks = nblocks_of(&c);
  p.eps = c.eps;
  p.attn_scale = (float)(1.0 / sqrt((double)c.HD));
  if (ds) {                                  // softmax_scale (reference_decode.py:198-206): q_head_dim^-0.5 * mscale^2
    const double mm = c.rope_factor <= 1.0f ? 1.0 : 0.1 * c.rope_mscale_all * log((double)c.rope_factor) + 1.0;
    p.attn_scale = (float)(pow((double)(c.qk_nope + c.qk_rope), -0.5) * mm * mm);
  }
  p.embed = (const uint16_t*)h->wt(ETXMK_T_EMBED, -1);
  p.lm_head = (const uint16_t*)h->wt(ETXMK_T_LMHEAD, -1);
  p.final_norm = (const uint16_t*)h->wt(ETXMK_T_FINAL_NORM, -1);
  p.layers = h->wsptr<const LayerW>(h->ws.layers);
  p.rope_cos = h->wsptr<const float>(h->ws.rcos);
  p.rope_sin = h->wsptr<const float>(h->ws.rsin);
  p.btab = h->wsptr<const int32_t>(h->ws.btab);
  p.x = h->wsptr<float>(h->ws.x);
  p.qkv = h->wsptr<float>(h->ws.qkv);
  p.o = h->wsptr<float>(h->ws.o);
  p.logits = h->wsptr<float>(h->ws.logits);
  p.hbuf = h->wsptr<float>(h->ws.hbuf);
  p.apart = h->wsptr<float>(h->ws.apart);
  p.acnt = h->wsptr<uint32_t>(h->ws.acnt);
  p.amax = h->wsptr<uint64_t>(h->ws.amax);
  p.bar = h->wsptr<uint32_t>(h->ws.bar);
  p.abort_word = h->wsptr<int32_t>(h->ws.abort_w);
  p.tokens = h->wsptr<int32_t>(h->ws.tokens);
  p.out_tokens = h->wsptr<int32_t>(h->ws.out_tokens);
  if (!pf) {                               // the dump buffers hold `batch` rows; prefill rows are not dumped
    p.dump_x = h->dump_x; p.dump_ids = h->dump_ids; p.dump_wts = h->dump_wts; p.dump_logits = h->dump_logits;
  }
  p.trace = h->fused && !pf ? h->trace : nullptr;   // the stamp buffer is sized for the handle's step kernel
  p.pos = batched ? 0 : pos; p.write_next = write_next; p.l0 = l0; p.l1 = l1; p.do_embed = embed; p.do_head = head;
  p.nwg = h->nwg;
  p.spin_ticks = h->spin_ticks;
  p.poll_mask = h->poll_mask;
  p.host_stop = h->stop_dev;
  {  // a workgroup's QKV rows: staged in LDS a layer ahead as far as the stage holds them, the rest (rows of 4096
     // only, up to two per wave) loaded into registers before the QKV phase's wait
    const int rows = nqkv_of(c), R = (rows + h->nwg - 1) / h->nwg;
    const int S = R < (int)(QKVW_BYTES / (2 * c.H)) ? R : (int)(QKVW_BYTES / (2 * c.H));
    const int regs = c.H >= 4096 ? 2 * NWAVE : 0;
    const bool ok = !batched && h->fused && c.wdtype == ETXMK_W_BF16 && c.H % 512 == 0 && R - S <= regs;
    p.qkv_rows = ok ? R : 0;
    p.qkv_lds_rows = ok ? S : 0;
  }
  p.B = nrows;
  p.mfma = mfma_rule(c);
  p.nbps = nbps_of(&c);
  p.tok_stride = c.max_ctx + 1;
  if (pf) {                                // every row reads the one sequence's block table and token rows
    p.pf = 1;
    p.btab += (size_t)pseq * p.nbps;
    p.tokens += (size_t)pseq * p.tok_stride;
    p.out_tokens += (size_t)pseq * p.tok_stride;
    p.nbps = 0;
    p.tok_stride = 0;
  }
  p.x16 = h->wsptr<uint16_t>(h->ws.x16);
  p.o16 = h->wsptr<uint16_t>(h->ws.o16);
  p.h16 = h->wsptr<uint16_t>(h->ws.h16);
  p.ys = h->wsptr<uint16_t>(h->ws.ys);
  p.nqkv = nqkv_of(c);
  p.Ip = ds ? ds_ip(c) : c.I;
  p.h16d = h->wsptr<uint16_t>(h->ws.h16d);
  p.sink = h->wsptr<float>(h->ws.sink);
  p.arch = c.arch;
  if (ds) {
    p.I = c.dense_I;
    p.first_dense = c.first_dense;
    p.SI = ds_si(c);
    p.routed_scale = c.routed_scale;
    p.qc = h->wsptr<float>(h->ws.qc);
    p.h16s = h->wsptr<uint16_t>(h->ws.h16s);
  }
  // attention items of each sequence: DeepSeek-V2 one per (group of 8 heads, 64-position chunk); Qwen3 one per
  // (kv head, ATTN_CPI_B chunks) in batched kernels (the single-sequence kernel counts its own, one chunk each)
  p.ibase[0] = 0;
  for (int b = 0; b < nrows; ++b) {
    p.posb[b] = batched ? posv[b] : pos;
    const int nch = p.posb[b] / CHUNK + 1;
    p.ibase[b + 1] = p.ibase[b] + (ds ? ds_nhg(c) * nch : c.NKV * ((nch + ATTN_CPI_B - 1) / ATTN_CPI_B));
  }
  if (h->fused) {
    // p.mfma launches take a kernel of capacity >= 8 whatever their row count (a short prefill included): the tile
    // forms exist in those kernels only, and the rule is the handle's, not the launch's
    const void* fn = ds ? ds_kernel(c) : batched ? batch_kernel(c, p.mfma && nrows < 8 ? 8 : nrows) : fused_kernel(c);
    if (!fn) return fail(ETXMK_EINVAL, "no persistent kernel for H %d, NH*HD %d, %s %d (use the unfused mode)", c.H,
                         c.NH * c.HD, c.moe ? "MI" : "I", c.moe ? c.MI : c.I);
    p.bar_base = h->bar_epoch;
    if (sv) {                              // scratch outside the workspace; its counters were cleared just before
      p.x = (float*)(sv->base + sv->lay.x);
      p.qkv = (float*)(sv->base + sv->lay.qkv);
      p.o = (float*)(sv->base + sv->lay.o);
      p.logits = (float*)(sv->base + sv->lay.logits);
      p.hbuf = (float*)(sv->base + sv->lay.hbuf);
      p.apart = (float*)(sv->base + sv->lay.apart);
      p.acnt = (uint32_t*)(sv->base + sv->lay.acnt);
      p.amax = (uint64_t*)(sv->base + sv->lay.amax);
      p.bar = (uint32_t*)(sv->base + sv->lay.bar);
      p.bar_base = 0;
    }
    void* args[] = {&p};
    HIPCHK(hipLaunchCooperativeKernel(fn, dim3(h->nwg), dim3(NT), args, 0, st));
    if (!sv) h->bar_epoch += (uint32_t)h->barriers(l0, l1, head, batched);
  } else {
    auto ph = [&](int phase, int layer) -> int {
      static void (*const kern[])(Params, int) = {etxmk_p_qkv, etxmk_p_attn, etxmk_p_oproj, etxmk_p_router,
                                                  etxmk_p_expert_up, etxmk_p_expert_down, etxmk_p_gateup,
                                                  etxmk_p_down, etxmk_p_head, etxmk_p_token};
      hipLaunchKernelGGL(kern[phase], dim3(h->nwg), dim3(NT), 0, st, p, layer);
      HIPCHK(hipGetLastError());
      return ETXMK_OK;
    };
    for (int l = l0; l < l1; ++l) {
      int r = ph(PH_QKV, l);
      r = r ? r : ph(PH_ATTN, l);
      r = r ? r : ph(PH_OPROJ, l);
      if (c.moe) {
        r = r ? r : ph(PH_ROUTER, l);
        r = r ? r : ph(PH_EXPUP, l);
        r = r ? r : ph(PH_EXPDN, l);
      } else {
        r = r ? r : ph(PH_GATEUP, l);
        r = r ? r : ph(PH_DOWN, l);
      }
      if (r) return r;
    }
    if (head) {
      if (int r = ph(PH_HEAD, 0)) return r;
      if (int r = ph(PH_TOKEN, 0)) return r;
    }
  }
  return ETXMK_OK;
}

int etxmk_step(etxmk_handle* h, int32_t pos, int32_t write_next, void* stream) {
  if (!h) return fail(ETXMK_EINVAL, "NULL handle");
  return launch(h, nullptr, pos, write_next, 0, h->c.L, 1, 1, (hipStream_t)stream);
}

int etxmk_step_static(etxmk_handle* h, int32_t pos, int32_t write_next, void* stream) {
  if (!h || !h->wsp) return fail(ETXMK_EUNBOUND, "handle not bound");
  const etxmk_config& c = h->c;
  if (c.batch != 1 || is_ds(c) || !h->fused)
    return fail(ETXMK_EINVAL, "etxmk_step_static runs single-sequence Qwen3 handles in fused mode");
  if (!fused_kernel(c)) return fail(ETXMK_EINVAL, "no persistent kernel for this shape");
  ScratchView sv{};
  sv.lay = static_layout(c);
  if (sv.lay.total > STATIC_SCRATCH_BYTES)
    return fail(ETXMK_EINVAL, "the step needs %llu bytes of scratch, above the %llu-byte static buffer",
                (unsigned long long)sv.lay.total, (unsigned long long)STATIC_SCRATCH_BYTES);
  if (int r = scratch_ptr(&sv.base)) return r;
  hipStream_t st = (hipStream_t)stream;
  // the counters must start at zero: a fill kernel (capturable), not a memset
  const size_t n16 = sv.lay.zero_end / 2;
  hipLaunchKernelGGL(etxmk_fill_u16, dim3(8), dim3(256), 0, st, (uint16_t*)(sv.base + sv.lay.bar), n16, (uint16_t)0);
  HIPCHK(hipGetLastError());
  return launch(h, nullptr, pos, write_next, 0, c.L, 1, 1, st, -1, 0, &sv);
}

int etxmk_step_batch(etxmk_handle* h, const int32_t* positions, int32_t write_next_mask, void* stream) {
  if (!h) return fail(ETXMK_EINVAL, "NULL handle");
  if (!positions) return fail(ETXMK_EINVAL, "positions is NULL");
  return launch(h, positions, 0, write_next_mask, 0, h->c.L, 1, 1, (hipStream_t)stream);
}

int etxmk_prefill(etxmk_handle* h, int32_t seq, int32_t pos0, int32_t n, int32_t write_next, void* stream) {
  if (!h) return fail(ETXMK_EINVAL, "NULL handle");
  const etxmk_config& c = h->c;
  if (!h->fused) return fail(ETXMK_EINVAL, "prefill runs the persistent kernel only");
  if (seq < 0 || seq >= c.batch) return fail(ETXMK_EINVAL, "sequence %d outside 0..%d", seq, c.batch - 1);
  if (n < 1 || n > rows_of(c)) return fail(ETXMK_EINVAL, "%d prefill positions outside 1..%d", n, rows_of(c));
  if (pos0 < 0 || pos0 + n > c.max_ctx)
    return fail(ETXMK_EINVAL, "positions %d..%d outside 0..%d", pos0, pos0 + n - 1, c.max_ctx - 1);
  if (!is_ds(c) && !batch_kernel(c, n))
    return fail(ETXMK_EINVAL, "no batched persistent kernel for %d rows, H %d, NH*HD %d, %s %d", n, c.H, c.NH * c.HD,
                c.moe ? "MI" : "I", c.moe ? c.MI : c.I);
  int32_t posv[MAX_B];
  for (int b = 0; b < n; ++b) posv[b] = pos0 + b;
  return launch(h, posv, 0, write_next ? 1 << (n - 1) : 0, 0, c.L, 1, 1, (hipStream_t)stream, seq, n);
}

int etxmk_step_layers(etxmk_handle* h, int32_t pos, int32_t l0, int32_t l1, void* stream) {
  if (!h) return fail(ETXMK_EINVAL, "NULL handle");
  if (h->c.batch != 1 || is_ds(h->c)) return fail(ETXMK_EINVAL, "layer-range steps serve single-sequence Qwen3 handles");
  return launch(h, nullptr, pos, 0, l0, l1, 0, 0, (hipStream_t)stream);
}

int etxmk_abort(etxmk_handle* h) {
  if (!h) return fail(ETXMK_EINVAL, "NULL handle");
  __atomic_store_n(h->stop_host, 1, __ATOMIC_SEQ_CST);
  return ETXMK_OK;
}

int etxmk_set_spin_limit(etxmk_handle* h, uint64_t ticks, int32_t check_every) {
  if (!h) return fail(ETXMK_EINVAL, "NULL handle");
  if (check_every == 0) check_every = 256;
  if (check_every < 1 || check_every > 256 || (check_every & (check_every - 1)))
    return fail(ETXMK_EINVAL, "check_every %d is not a power of two in 1..256", check_every);
  h->spin_ticks = ticks ? ticks : SPIN_TICKS_DEFAULT;
  h->poll_mask = (uint32_t)check_every - 1u;
  return ETXMK_OK;
}

int etxmk_sync_timeout(etxmk_handle* h, void* stream, int64_t timeout_ms) {
  if (!h || !h->wsp) return fail(ETXMK_EUNBOUND, "handle not bound");
  hipStream_t st = (hipStream_t)stream;
  bool timed_out = false;
  if (timeout_ms >= 0) {
    // poll the stream; past the limit ask the running step to stop (its waits read the stop word) and let it drain
    const auto t0 = std::chrono::steady_clock::now();
    for (;;) {
      const hipError_t q = hipStreamQuery(st);
      if (q == hipSuccess) break;
      if (q != hipErrorNotReady) return fail(ETXMK_EHIP, "hipStreamQuery: %s", hipGetErrorString(q));
      if (std::chrono::steady_clock::now() - t0 >= std::chrono::milliseconds(timeout_ms)) {
        timed_out = true;
        __atomic_store_n(h->stop_host, 1, __ATOMIC_SEQ_CST);
        break;
      }
      std::this_thread::yield();
    }
  }
  const hipError_t e = hipStreamSynchronize(st);
  __atomic_store_n(h->stop_host, 0, __ATOMIC_SEQ_CST);   // the stream has drained: no step can read it any more
  if (e != hipSuccess) return fail(ETXMK_EHIP, "hipStreamSynchronize: %s", hipGetErrorString(e));
  int32_t ab = 0;
  HIPCHK(hipMemcpy(&ab, h->wsp + h->ws.abort_w, 4, hipMemcpyDeviceToHost));
  if (ab) {
    HIPCHK(hipMemset(h->wsp + h->ws.abort_w, 0, 4));
    HIPCHK(hipMemset(h->wsp + h->ws.bar, 0, 4 * 64 * 17));
    HIPCHK(hipMemset(h->wsp + h->ws.acnt, 0, acnt_bytes(h->c)));
    h->bar_epoch = 0;
    if (timed_out)
      return fail(ETXMK_TIMEOUT, "the stream was still running after %lld ms; the step was stopped (abort word %d)",
                  (long long)timeout_ms, ab);
    return fail(ETXMK_ABORTED, "device abort word %d (%s)", ab,
                ab == 2 ? "a grid barrier wait exceeded its limit" : ab == 3 ? "no finite logit in the head" : "host stop");
  }
  if (timed_out)   // the step finished on its own before any wait saw the stop request: its results stand
    return fail(ETXMK_TIMEOUT, "the stream was still running after %lld ms (it completed before the stop was seen)",
                (long long)timeout_ms);
  return ETXMK_OK;
}

int etxmk_sync(etxmk_handle* h, void* stream) { return etxmk_sync_timeout(h, stream, -1); }

}  // extern "C"
