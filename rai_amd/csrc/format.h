// .raimodel reader: validation and section views over a host image.
// Restates rai-infer/src/format.rs (header 1098-1365, config 1376-1480,
// layout 557-1082, parameter checks 1492-1521) for the capability subset
// this build implements.
#ifndef RAI_FORMAT_H
#define RAI_FORMAT_H

#include <cstdint>
#include <string>
#include <vector>

#include "common.h"

namespace rai {

// Byte range of one quantized linear inside the image:
// [u32 rows][u32 cols][rows*groups*4 params][rows*cols/2 nibbles].
struct LinearView {
  uint32_t rows = 0, cols = 0, group_size = 0;
  size_t params_off = 0, params_len = 0;
  size_t nib_off = 0, nib_len = 0;
};

struct LayerView {
  LinearView lin[7];                // q k v o gate up down (format.rs:86-94)
  std::vector<LinearView> experts;  // experts 1..E-1, 3 linears each (gate, up, down)
  size_t router_off = 0;            // f32 [E][hidden], when MoE
  size_t in_norm_off = 0, post_norm_off = 0;  // f32 [hidden]
};

struct ModelView {
  rai_model_config cfg{};
  size_t header_size = 0;
  std::vector<std::pair<uint64_t, uint64_t>> sections;
  size_t emb_params_off = 0, emb_codes_off = 0;
  std::vector<LayerView> layers;
  size_t final_norm_off = 0;
  bool tied = false;
  LinearView lm_head;
  float attention_scale = 0.0f;
};

// Parse and validate a complete image (RaiModelFile::open).  max_groups = 0
// means the reference's MAX_GROUPS (128).  Throws rai::Error.
ModelView parse_model(const uint8_t *data, size_t len, int max_groups);

float f16_bits_to_f32(uint16_t h);

}  // namespace rai

#endif
