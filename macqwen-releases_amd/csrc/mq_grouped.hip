// Prefill / verify grouped path (token-sorted gather_qmm with bf16 MFMA).
#include "mq_internal.h"

using namespace mq;

extern "C" uint64_t mq_grouped_workspace_size(uint32_t tokens, uint32_t slots, uint32_t hidden,
                                              uint32_t inter, uint32_t expert_count) {
  (void)tokens; (void)slots; (void)hidden; (void)inter; (void)expert_count;
  return 0;
}

extern "C" int mq_moe_grouped(const MqGroupedArgs *args, void *stream) {
  (void)args; (void)stream;
  return fail(MQ_ERR_UNSUPPORTED, "grouped path not built yet");
}
