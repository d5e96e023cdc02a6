/**
 * forge-llm_amd · public API of the MI355X training path: the same names as
 * forge-llm's src/index.js for the tensor ops, autograd, Config and the
 * trainable model.
 */
export { RNG, maxAbsErr, rmse, relL2, cosSim } from "./L0/numeric.js";
export {
  Node, leaf, param, op, tape, resetTape, noGrad, linear, add, mul, silu as siluAD, rmsnorm as rmsnormAD,
  softmaxCE, backward, gradCheck, Adam, dot as dotAD, scale as scaleAD, ropeNode, softmaxVec,
} from "./L2/autograd.js";
export {
  matmulT, matmul, embedLookup, rmsNorm, ropeRows, sliceCols, causalAttn, causalAttnBatch, swigluRows,
  crossEntropyMean, crossEntropyMeanFused, weightedSum, qkvRope, qkvRopeAttention, matmulTResid, swigluGateUp,
  packPair, DeviceIds,
} from "./L2/tensor.js";
export { Config, Transformer } from "./L6/transformer.js";
export { KVCache, attentionDecode, attentionNaive, flashAttention } from "./L5/attention.js";
export { TrainableTransformer, initWeights, toParams, train, DeviceTrainLoop } from "./L6/train.js";
export { hip } from "./L2/device.js";
export {
  dequantize, quantizeRow, dotQ, rowBytes, info, qualityReport, TYPE_INFO, TYPE_NAME, GGMLType, QK_K, fp16Table,
  quantizeRowQ4K, quantizeRowQ5K, quantizeRowQ6K, quantizeRowQ8_0, quantizeRowF16,
} from "./L3/quant.js";
export { QuantLinear, SwiGLU, rmsnormInto } from "./L4/nn.js";
export { writeGGUF, readGGUF, GGUFValueType, tensorBytes, ggmlTypeSize } from "./L9/gguf.js";
export { exportGGUF, loadGGUF, saveCheckpoint, loadCheckpoint } from "./L9/export.js";
