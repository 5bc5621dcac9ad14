'use strict';
// Entry point of the TypeScript host checks: registers the .ts loader, then runs selftest.ts.
//   node gemma4-webgpu_amd/host/run.js cpu | layer <dir>
require('./ts_register').register();
try {
  require('./selftest.ts').main(process.argv.slice(2));
} catch (e) {
  process.stderr.write(String(e && e.stack ? e.stack : e) + '\n');
  process.exit(1);
}
