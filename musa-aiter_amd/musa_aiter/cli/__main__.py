from musa_aiter.cli.main import main

raise SystemExit(main())
