// Minimal test runner for Node 12 (no node:test): test(name, fn) collects,
// run() executes in order, prints one JSON line per test and exits non-zero
// if any failed.
const _tests = [];
export function test(name, fn) { _tests.push({ name, fn }); }
export function assert(cond, msg) { if (!cond) throw new Error(msg || "assertion failed"); }
export async function run() {
  const only = process.argv[2] || null;
  let failed = 0;
  for (const t of _tests) {
    if (only && !t.name.includes(only)) continue;
    const t0 = Date.now();
    try {
      const detail = await t.fn();
      console.log(JSON.stringify({ test: t.name, ok: true, ms: Date.now() - t0, detail: detail === undefined ? null : detail }));
    } catch (e) {
      failed++;
      console.log(JSON.stringify({ test: t.name, ok: false, ms: Date.now() - t0, error: String(e && e.stack || e) }));
    }
  }
  process.exit(failed ? 1 : 0);
}
