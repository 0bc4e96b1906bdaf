// Per-layer shape of the qwen35moe 35B-A3B model the kernels are specialised for (BASELINE shape;
// the reference reads the same numbers from GGUF metadata, crates/model/src/desc.rs:69-140). The
// layer count, vocabulary and context are runtime values; the engine refuses any other per-layer
// shape at creation.
#pragma once

namespace oxe {
namespace shp {
constexpr int E = 2048;        // n_embd
constexpr int NH = 16;         // query heads
constexpr int NKV = 2;         // kv heads
constexpr int HD = 256;        // head_dim
constexpr int GQA = NH / NKV;  // query heads per kv head
constexpr int NEXP = 256;      // routed experts
constexpr int KUSED = 8;       // experts per token
constexpr int FF = 512;        // expert FFN width
constexpr int FFSH = 512;      // shared expert FFN width
constexpr int KC = 4;          // conv kernel
constexpr int DS = 128;        // delta-net key head dim
constexpr int NKH = 16;        // delta-net key heads
constexpr int NVH = 32;        // delta-net value heads
constexpr int HV = 128;        // delta-net value head dim
constexpr int DIN = NVH * HV;  // 4096
constexpr int NCH = DIN + 2 * NKH * DS;  // conv channels 8192
constexpr int NROT = 64;       // rotated dims
// delta-net projection rows [qkv | z | beta | alpha]
constexpr int DN_Z = NCH, DN_BETA = NCH + DIN, DN_ALPHA = DN_BETA + NVH, DN_ROWS = DN_ALPHA + NVH;  // 12352
// attention projection rows [q+gate per head | k | v]
constexpr int AT_K = NH * 2 * HD, AT_V = AT_K + NKV * HD, AT_ROWS = AT_V + NKV * HD;               // 9216
constexpr int MIX_W = 4096;    // mixer output width (d_inner = n_head * head_dim = 4096)
}  // namespace shp
}  // namespace oxe
