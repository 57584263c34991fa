// A minimal test runner for Node 12 (no node:test): test(name, fn) registers
// a case, run() executes them in order, prints one line per case and sets the
// exit code to 1 if any failed.
const cases = [];
export function test(name, fn) { cases.push({name, fn}); }
export async function run() {
    let failed = 0;
    for (const c of cases) {
        try { await c.fn(); console.log('ok   ' + c.name); }
        catch (error) { failed++; console.log('FAIL ' + c.name + '\n     ' + (error && error.stack || error)); }
    }
    console.log(cases.length - failed + '/' + cases.length + ' passed');
    process.exitCode = failed ? 1 : 0;
}
