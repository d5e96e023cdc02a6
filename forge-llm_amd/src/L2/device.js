/**
 * Loader of the HIP addon (forge-llm_amd/lib/forge_napi.node → libforge_hip.so).
 *
 * There is no CPU fallback: if the addon cannot be loaded or no GPU is visible,
 * the first op throws.  FORGE_ADDON overrides the addon path, FORGE_DEVICE the
 * device index.
 */
import { createRequire } from "module";
import { fileURLToPath } from "url";
import { dirname, join } from "path";

const HERE = dirname(fileURLToPath(import.meta.url));
const requireNative = createRequire(import.meta.url);
let _addon = null;

/** The addon, initialised on the selected device (throws when unavailable). */
export function hip() {
  if (_addon) return _addon;
  const path = process.env.FORGE_ADDON || join(HERE, "..", "..", "lib", "forge_napi.node");
  let a;
  try {
    a = requireNative(path);
  } catch (e) {
    throw new Error(`forge-llm_amd: HIP addon not loadable from ${path} (build it with forge-llm_amd/build.py): ${e.message}`);
  }
  const dev = process.env.FORGE_DEVICE ? parseInt(process.env.FORGE_DEVICE, 10) : 0;
  a.init(dev);
  _addon = a;
  return a;
}

/** The addon without initialising a device (for introspection on GPU-less hosts). */
export function addonUninitialised() {
  const path = process.env.FORGE_ADDON || join(HERE, "..", "..", "lib", "forge_napi.node");
  return requireNative(path);
}

/** Allocate a device buffer of n fp32 elements (at least one). */
export function allocF32(n) {
  return hip().alloc(Math.max(1, n) * 4);
}

/** True while a step is being recorded into a graph (forge-llm_amd/src/L6/
 *  train.js): ops then queue no host read-backs, which a graph cannot hold. */
export const graphState = { capturing: false };
