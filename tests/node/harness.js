"use strict";
/* A small sequential test runner for the Node host tests: prints one line per
 * test and exits non-zero when any test fails. */
const tests = [];

function test(name, fn) {
  tests.push({ name, fn });
}

function run() {
  let failed = 0;
  for (const t of tests) {
    const t0 = Date.now();
    try {
      const skipped = t.fn();
      if (skipped === "skip") console.log("skip " + t.name);
      else console.log("ok   " + t.name + " (" + (Date.now() - t0) + " ms)");
    } catch (error) {
      failed += 1;
      console.log("FAIL " + t.name + "\n" + (error && error.stack ? error.stack : error));
    }
  }
  console.log(failed ? failed + " failed of " + tests.length : "all " + tests.length + " passed");
  process.exitCode = failed ? 1 : 0;
}

module.exports = { test, run };
