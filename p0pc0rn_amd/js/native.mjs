// native.mjs - loads the N-API addon (p0pc0rn.node, built by `python -m p0pc0rn_amd.build napi`). There is no fallback:
// without the addon the host cannot run, and it says so.
import { createRequire } from 'module';

const require = createRequire(import.meta.url);
let addon = null, loadError = null;
try {
  addon = require('./p0pc0rn.node');
} catch (e) {
  loadError = e;
}

/** the addon, or a thrown Error naming what is missing */
export function native() {
  if (!addon) throw new Error('p0pc0rn: the HIP addon is not built or failed to load (python -m p0pc0rn_amd.build): ' + (loadError && loadError.message));
  return addon;
}
